// W4 group-quantized GEMV for one decode token, with its fused prologue/epilogues.
//
// Semantics follow the reference's packed GEMV (codegen/matmul.py:542-739):
//   y[n] = sum_k code[n,k] * x[k] * s[n, k/group]       (f32 accumulation)
// with an optional RMSNorm prologue x' = bf16(ns * x * w), an addmm epilogue
// bf16(beta * bias[n] + alpha * acc), or the paired gate/up epilogue
// bf16(acc_up * g / (1 + exp(-g))), g = bf16(acc_gate).
//
// CDNA4 design (HBM-bound; the int4 decode must stay under the VALU budget):
// * The block stages x once in LDS as bf16 pairs (x[k], x[k+4]) per packed
//   word, plus one f32 sum of x per 32-code chunk.
// * `LPR` lanes share an output row; each lane streams whole 16-byte chunks
//   (4 words = 32 codes, one global_load_dwordx4) of that row, `U` chunks in
//   flight per lane, so a wave keeps U KiB of weights outstanding.
// * Nibbles become bf16 without a convert: (w ^ 0x88888888) puts code+8 in each
//   nibble; OR-ing two nibbles under 0x4300 gives the bf16 pair (136+c_a,
//   136+c_b), and v_dot2_f32_bf16 multiplies it with the matching x pair into an
//   f32 accumulator. Per word: 1 xor, 3 shifts, 4 and-or, 4 dot2 = 1.5 VALU ops
//   per weight. The +136 offset is removed once per chunk with the staged sum:
//   sum (136+c) x = sum c x + 136 sum x. Every product is exact in f32.
// * The group scale multiplies the chunk sum (group % 32 == 0, so a chunk never
//   straddles two groups); lanes of a row combine with a shuffle tree.
#pragma once

#include "common.h"

namespace aoto {

constexpr int kGemvThreads = 256;

// One 32-code chunk: dot of (136 + code) with x over 4 words, f32.
AOTO_DEVICE float chunk_dot(const uint4 q, const uint4* __restrict__ xc) {
  const uint32_t words[4] = {q.x, q.y, q.z, q.w};
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t t = words[j] ^ 0x88888888u;
    const uint4 xv = xc[j];
    acc = dot2_bf16((t & 0x000F000Fu) | 0x43004300u, xv.x, acc);
    acc = dot2_bf16(((t >> 4) & 0x000F000Fu) | 0x43004300u, xv.y, acc);
    acc = dot2_bf16(((t >> 8) & 0x000F000Fu) | 0x43004300u, xv.z, acc);
    acc = dot2_bf16(((t >> 12) & 0x000F000Fu) | 0x43004300u, xv.w, acc);
  }
  return acc;
}

// Stage x (optionally RMS-normalized and rounded to bf16) into LDS in dot2 pair
// order, plus per-chunk sums. Ends with a barrier.
template <bool NORM>
AOTO_DEVICE void stage_activation(const uint16_t* __restrict__ x, const uint16_t* __restrict__ norm_w,
                                  float eps, int K, uint4* __restrict__ xp, float* __restrict__ csum,
                                  float* __restrict__ scratch) {
  const int nchunks = K >> 5;
  float ns = 1.f;
  if (NORM) {
    float ss = 0.f;
    const uint4* xv = reinterpret_cast<const uint4*>(x);
    for (int i = threadIdx.x; i < (K >> 3); i += kGemvThreads) {
      const uint4 r = xv[i];
      const uint32_t v[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = bf16_lo(v[j]), b = bf16_hi(v[j]);
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
    }
    ss = block_sum<kGemvThreads>(ss, scratch);
    ns = 1.0f / sqrtf(ss / (float)K + eps);
  }
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  const uint4* wv = reinterpret_cast<const uint4*>(norm_w);
  for (int c = threadIdx.x; c < nchunks; c += kGemvThreads) {
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 r = xv[c * 4 + j];
      const uint32_t raw[4] = {r.x, r.y, r.z, r.w};
      float v[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16_lo(raw[i]);
        v[2 * i + 1] = bf16_hi(raw[i]);
      }
      if (NORM) {
        const uint4 wr = wv[c * 4 + j];
        const uint32_t wraw[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[2 * i] = round_bf16((ns * v[2 * i]) * bf16_lo(wraw[i]));
          v[2 * i + 1] = round_bf16((ns * v[2 * i + 1]) * bf16_hi(wraw[i]));
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) sum += v[i];
      uint4 out;
      out.x = pack_bf16x2(v[0], v[4]);
      out.y = pack_bf16x2(v[1], v[5]);
      out.z = pack_bf16x2(v[2], v[6]);
      out.w = pack_bf16x2(v[3], v[7]);
      xp[c * 4 + j] = out;
    }
    csum[c] = sum;
  }
  __syncthreads();
}

template <int LPR, int U, bool NORM, bool PAIRED, bool BIAS>
__device__ void w4_gemv_body(const uint16_t* __restrict__ x, const uint4* __restrict__ words,
                             const uint16_t* __restrict__ scales, const uint4* __restrict__ up_words,
                             const uint16_t* __restrict__ up_scales, const uint16_t* __restrict__ norm_w,
                             float eps, const uint16_t* __restrict__ bias, float alpha, float beta,
                             uint16_t* __restrict__ y, int K, int N, int group) {
  extern __shared__ uint4 lds[];
  __shared__ float scratch[kGemvThreads / 64];
  const int nchunks = K >> 5;
  uint4* xp = lds;
  float* csum = reinterpret_cast<float*>(lds + (K >> 3));
  stage_activation<NORM>(x, norm_w, eps, K, xp, csum, scratch);

  constexpr int kRowsPerWave = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & (LPR - 1);
  const int row = (blockIdx.x * (kGemvThreads / 64) + wave) * kRowsPerWave + lane / LPR;
  const bool active = row < N;
  const int r = active ? row : 0;
  const int ngroups = K / group;
  const int chunks_per_group = group >> 5;
  const uint4* wrow = words + (size_t)r * nchunks;
  const uint16_t* srow = scales + (size_t)r * ngroups;
  const uint4* urow = PAIRED ? up_words + (size_t)r * nchunks : nullptr;
  const uint16_t* usrow = PAIRED ? up_scales + (size_t)r * ngroups : nullptr;

  float total = 0.f, total_up = 0.f;
  for (int c0 = li; c0 < nchunks; c0 += LPR * U) {
    uint4 q[U];
    uint4 qu[PAIRED ? U : 1];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * LPR;
      if (c < nchunks) {
        q[u] = wrow[c];
        if (PAIRED) qu[u] = urow[c];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * LPR;
      if (c < nchunks) {
        const uint4* xc = xp + c * 4;
        const float corr = 136.f * csum[c];
        const int g = c / chunks_per_group;
        total = fmaf(chunk_dot(q[u], xc) - corr, bf16_to_f32(srow[g]), total);
        if (PAIRED) total_up = fmaf(chunk_dot(qu[u], xc) - corr, bf16_to_f32(usrow[g]), total_up);
      }
    }
  }
  total = group_sum<LPR>(total);
  if (PAIRED) total_up = group_sum<LPR>(total_up);
  if (active && li == 0) {
    float out;
    if (PAIRED) {
      const float g = round_bf16(total);
      out = total_up * (g / (1.0f + expf(-g)));
    } else if (BIAS) {
      out = beta * bf16_to_f32(bias[row]) + alpha * total;
    } else {
      out = total;
    }
    y[row] = (uint16_t)f32_to_bf16(out);
  }
}

}  // namespace aoto

#define AOTO_GEMV_INSTANCE(LPR, NORM, PAIRED, BIAS)                                              \
  extern "C" __global__ __launch_bounds__(aoto::kGemvThreads) void                               \
      aoto_w4_gemv_l##LPR##_n##NORM##_p##PAIRED##_b##BIAS(                                       \
          const uint16_t* x, const uint4* words, const uint16_t* scales, const uint4* up_words,   \
          const uint16_t* up_scales, const uint16_t* norm_w, float eps, const uint16_t* bias,     \
          float alpha, float beta, uint16_t* y, int K, int N, int group) {                       \
    aoto::w4_gemv_body<LPR, 4, NORM, PAIRED, BIAS>(x, words, scales, up_words, up_scales, norm_w, \
                                                   eps, bias, alpha, beta, y, K, N, group);      \
  }

#define AOTO_GEMV_LPR(NORM, PAIRED, BIAS)   \
  AOTO_GEMV_INSTANCE(4, NORM, PAIRED, BIAS)  \
  AOTO_GEMV_INSTANCE(8, NORM, PAIRED, BIAS)  \
  AOTO_GEMV_INSTANCE(16, NORM, PAIRED, BIAS) \
  AOTO_GEMV_INSTANCE(32, NORM, PAIRED, BIAS) \
  AOTO_GEMV_INSTANCE(64, NORM, PAIRED, BIAS)
