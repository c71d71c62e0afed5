// Symmetric int8 group quantization: packer, bf16 unpack and the decode GEMV.
//
// Restates quantize.py:155-172, 216-268 and models/quantized.py:84-107, 165-172
// of the reference (its eight-bit width, same skeleton as int4):
//   scale = max|w| / 127 in f32 (an all-zero group takes 1/127);
//   code  = clip(rint(w / scale), -128, 127), IEEE f32 division, half-to-even;
//   word j of a row holds codes 4j..4j+3, code 4j+k in byte k (bits 8k);
//   the stored scale is bf16(scale) (RNE) while the codes use the f32 scale.
// The unpack writes bf16(code * scale_bf16). The GEMV keeps the int4 kernel's
// rounding points (codegen/matmul.py:742-929): code * (x * s) is exact in f32
// (8 + 8 + 8 bits), accumulation in f32, one rounding after the epilogue.
#pragma once

#include "common.h"
#include "w4_gemv.h"

namespace aoto {

// One thread per (row, group). `src_f32` selects an f32 source, else bf16.
extern "C" __global__ __launch_bounds__(256) void aoto_w8_quantize(
    const void* __restrict__ src, int src_f32, int rows, int inner, int group,
    int32_t* __restrict__ packed, uint16_t* __restrict__ scales_bf16, float* __restrict__ scales_f32) {
  const int groups = inner / group;
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long long)rows * groups) return;
  const int row = (int)(gid / groups);
  const int g = (int)(gid - (long long)row * groups);
  const size_t base = (size_t)row * inner + (size_t)g * group;
  auto load = [&](int i) -> float {
    if (src_f32) return reinterpret_cast<const float*>(src)[base + i];
    return bf16_to_f32(reinterpret_cast<const uint16_t*>(src)[base + i]);
  };
  float widest = 0.f;
  for (int i = 0; i < group; ++i) widest = fmaxf(widest, fabsf(load(i)));
  const float scale = (widest > 0.f ? widest : 1.0f) / 127.0f;
  int32_t* out = packed + (size_t)row * (inner >> 2) + (size_t)g * (group >> 2);
  for (int w = 0; w < (group >> 2); ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float code = rintf(load(w * 4 + k) / scale);
      code = fminf(fmaxf(code, -128.0f), 127.0f);
      word |= ((uint32_t)(int)code & 0xFFu) << (8 * k);
    }
    out[w] = (int32_t)word;
  }
  scales_bf16[(size_t)row * groups + g] = (uint16_t)f32_to_bf16(scale);
  if (scales_f32) scales_f32[(size_t)row * groups + g] = scale;
}

// One thread per packed word: four bf16(code * scale) values, one 8-byte store.
extern "C" __global__ __launch_bounds__(256) void aoto_w8_dequantize(
    const int32_t* __restrict__ packed, const uint16_t* __restrict__ scales, int rows, int inner,
    int group, uint16_t* __restrict__ out) {
  const int words = inner >> 2;
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long long)rows * words) return;
  const int row = (int)(gid / words);
  const int w = (int)(gid - (long long)row * words);
  const uint32_t word = (uint32_t)packed[gid];
  const float s = bf16_to_f32(scales[(size_t)row * (inner / group) + (w * 4) / group]);
  uint32_t v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int code = (int)(word << (24 - 8 * k)) >> 24;
    v[k] = f32_to_bf16((float)code * s);
  }
  reinterpret_cast<uint2*>(out)[gid] = make_uint2(v[0] | (v[1] << 16), v[2] | (v[3] << 16));
}

// Dot of one 16-byte chunk (16 int8 codes, 4 words) with its 16 x values.
// Flipping the sign bit of each byte gives u = code + 128 in 0..255; the byte
// converts straight to an exact f32 (v_cvt_f32_ubyte*), whose upper half is
// the exact bf16 of u, and two of them form one bf16 pair for v_dot2 against
// the naturally ordered x pair. The +128 comes off once per chunk with the
// staged x sum: sum code*x = sum u*x - 128 sum x. Every product is exact.
AOTO_DEVICE uint32_t byte_pair(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

AOTO_DEVICE float chunk_dot_w8(const uint4 q, const uint4* __restrict__ xc) {
  const uint32_t words[4] = {q.x, q.y, q.z, q.w};
  const uint4 xa = xc[0], xb = xc[1];
  const uint32_t xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t t = words[j] ^ 0x80808080u;
    const float u0 = (float)(t & 0xFFu), u1 = (float)((t >> 8) & 0xFFu);
    const float u2 = (float)((t >> 16) & 0xFFu), u3 = (float)(t >> 24);
    acc = dot2_bf16(byte_pair(u0, u1), xs[2 * j], acc);
    acc = dot2_bf16(byte_pair(u2, u3), xs[2 * j + 1], acc);
  }
  return acc;
}

// Decode GEMV over eight-bit words: y[n] = epilogue(sum_k code[n,k] * x'[k] * s[n,k/g]).
// x (RMS-normalized and rounded to bf16 with NORM, as the int4 GEMV does) is
// staged once per block in LDS in natural order, plus one f32 sum per 16-code
// chunk. A wave owns R output rows at a time; its 64 lanes stride over the
// rows' chunks, U chunks of each row per lane per pass, all R*U loads issued
// before any arithmetic. Waves are persistent over rows.
template <int R, int U, bool NORM, bool PAIRED, bool BIAS>
__device__ void w8_gemv_body(const uint16_t* __restrict__ x, const uint4* __restrict__ words,
                             const uint16_t* __restrict__ scales, const uint4* __restrict__ up_words,
                             const uint16_t* __restrict__ up_scales, const uint16_t* __restrict__ norm_w,
                             float eps, const uint16_t* __restrict__ bias, float alpha, float beta,
                             uint16_t* __restrict__ y, int K, int N, int group) {
  extern __shared__ uint4 lds[];
  __shared__ float scratch[kGemvThreads / 64];
  const int nchunks = K >> 4;
  uint4* xs = lds;                                            // [nchunks][2]
  float* csum = reinterpret_cast<float*>(lds + 2 * nchunks);  // [nchunks]
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  const uint4* wv = reinterpret_cast<const uint4*>(norm_w);

  float ns = 1.f;
  if (NORM) {
    float ss = 0.f;
    for (int v = threadIdx.x; v < (K >> 3); v += kGemvThreads) {
      const uint4 r = xv[v];
      const uint32_t raw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = bf16_lo(raw[j]), b = bf16_hi(raw[j]);
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
    }
    ss = block_sum<kGemvThreads>(ss, scratch);
    ns = 1.0f / sqrtf(ss / (float)K + eps);
  }
  // Thread v stages elements 8v..8v+7 (half of chunk v/2); K/8 is even, so the
  // two halves of a chunk are adjacent lanes of one iteration.
  for (int v = threadIdx.x; v < (K >> 3); v += kGemvThreads) {
    const uint4 r = xv[v];
    const uint32_t raw[4] = {r.x, r.y, r.z, r.w};
    float e[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      e[2 * j] = bf16_lo(raw[j]);
      e[2 * j + 1] = bf16_hi(raw[j]);
    }
    if (NORM) {
      const uint4 wq = wv[v];
      const uint32_t wr[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        e[2 * j] = round_bf16((ns * e[2 * j]) * bf16_lo(wr[j]));
        e[2 * j + 1] = round_bf16((ns * e[2 * j + 1]) * bf16_hi(wr[j]));
      }
    }
    xs[v] = make_uint4(pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3]), pack_bf16x2(e[4], e[5]),
                       pack_bf16x2(e[6], e[7]));
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += e[j];
    sum += __shfl_xor(sum, 1, 64);
    if ((v & 1) == 0) csum[v >> 1] = sum;
  }
  __syncthreads();

  const int groups = K / group;
  const int total_waves = gridDim.x * (kGemvThreads / 64);
  for (int row0 = (blockIdx.x * (kGemvThreads / 64) + wave) * R; row0 < N; row0 += total_waves * R) {
    float acc[R], acc_up[R];
    int rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc[r] = 0.f;
      acc_up[r] = 0.f;
      rows[r] = min(row0 + r, N - 1);  // rows past N repeat row N-1 and are not stored
    }
    for (int c0 = 0; c0 < nchunks; c0 += 64 * U) {
      uint4 q[R][U], qu[PAIRED ? R : 1][PAIRED ? U : 1];
      float s[R][U], su[PAIRED ? R : 1][PAIRED ? U : 1];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = min(c0 + u * 64 + lane, nchunks - 1);
          q[r][u] = words[(size_t)rows[r] * nchunks + c];
          if (PAIRED) qu[r][u] = up_words[(size_t)rows[r] * nchunks + c];
        }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = min(c0 + u * 64 + lane, nchunks - 1);
          const size_t si = (size_t)rows[r] * groups + (c << 4) / group;
          s[r][u] = bf16_to_f32(scales[si]);
          if (PAIRED) su[r][u] = bf16_to_f32(up_scales[si]);
        }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * 64 + lane;
        if (c < nchunks) {
          const float off = 128.f * csum[c];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            acc[r] = fmaf(chunk_dot_w8(q[r][u], xs + 2 * c) - off, s[r][u], acc[r]);
            if (PAIRED) acc_up[r] = fmaf(chunk_dot_w8(qu[r][u], xs + 2 * c) - off, su[r][u], acc_up[r]);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float total = wave_sum(acc[r]);
      const float total_up = PAIRED ? wave_sum(acc_up[r]) : 0.f;
      const int row = row0 + r;
      if (lane == 0 && row < N) {
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
  }
}

}  // namespace aoto

#define AOTO_GEMV_W8_INSTANCE(R, U, NORM, PAIRED, BIAS)                                                    \
  extern "C" __global__ __launch_bounds__(aoto::kGemvThreads) void                                         \
      aoto_w8_gemv_r##R##u##U##_n##NORM##_p##PAIRED##_b##BIAS(                                             \
          const uint16_t* x, const uint4* words, const uint16_t* scales, const uint4* up_words,           \
          const uint16_t* up_scales, const uint16_t* norm_w, float eps, const uint16_t* bias, float alpha, \
          float beta, uint16_t* y, int K, int N, int group) {                                             \
    aoto::w8_gemv_body<R, U, NORM, PAIRED, BIAS>(x, words, scales, up_words, up_scales, norm_w, eps, bias, \
                                                 alpha, beta, y, K, N, group);                            \
  }

// The decoder's epilogues for one (rows, chunks) shape.
#define AOTO_GEMV_W8_SHAPE(R, U)          \
  AOTO_GEMV_W8_INSTANCE(R, U, 0, 0, 0)    \
  AOTO_GEMV_W8_INSTANCE(R, U, 0, 0, 1)    \
  AOTO_GEMV_W8_INSTANCE(R, U, 1, 0, 0)    \
  AOTO_GEMV_W8_INSTANCE(R, U, 1, 0, 1)    \
  AOTO_GEMV_W8_INSTANCE(R, U, 1, 1, 0)    \
  AOTO_GEMV_W8_INSTANCE(R, U, 0, 1, 0)
