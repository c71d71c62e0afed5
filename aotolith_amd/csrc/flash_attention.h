// Prefill GQA attention on bf16 MFMA (online softmax, one pass over K/V).
//
// Semantics (runtime/mlx_ops/attention.py:73-122, legalize/attention.py:105-170,
// mask from models/decoder.py:226-247):
//   O[b][i][h*D:(h+1)*D] = sum_j softmax_j(scale * q_i . k_j | keep(i, j)) v_j
// with key/value head h / (Hq/Hkv), f32 scores and softmax, and a query row
// whose keys are all masked giving 0 (safe_softmax).
// keep(i, j): with `mask` non-null, mask[b*mask_batch_stride + i*Mk + j] != 0;
// otherwise j >= key_start and, when `causal`, j <= i + (Mk - M) - the
// reference's prefill mask "causal and not a left pad" at key_start = M - length.
//
// Layout: q[B][Hq][M][D] (head-major, as the fused RoPE writes it); keys and
// values at k/v + b*kv_batch_stride + kvh*kv_head_stride + j*D; output
// [B][M][Hq*D] (the o projection's input rows).
//
// Block: 4 waves x 16 queries = 64 queries of one head; key tiles of 64 staged
// in LDS (K row-major, V transposed). Per wave and key tile:
//   S^T (16 keys x 16 queries) = K . Q^T   v_mfma_f32_16x16x32_bf16, Q in registers
//   O^T (16 d x 16 queries)  += V^T . P^T  v_mfma_f32_16x16x16_bf16, P from S^T's registers
// In both products lane l owns query l%16 of its accumulators, so the running
// max/sum of that query live in the lane that rescales its O^T columns.
#pragma once

#include "common.h"

namespace aoto {

typedef __bf16 fa_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 fa_bf16x4 __attribute__((ext_vector_type(4)));
typedef float fa_f32x4 __attribute__((ext_vector_type(4)));

template <int D>
__device__ void flash_attention_body(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                     const uint16_t* __restrict__ v, long long kv_batch_stride,
                                     long long kv_head_stride, const uint8_t* __restrict__ mask,
                                     long long mask_batch_stride, int causal, int key_start, int M, int Mk,
                                     int query_heads, int kv_heads, float scale, uint16_t* __restrict__ out) {
  constexpr int BKV = 64;
  constexpr int KSTR = D + 8;       // bf16 per K row in LDS
  constexpr int VSTR = BKV + 8;     // bf16 per V^T row in LDS
  constexpr int DT = D / 16;        // d tiles of O^T
  constexpr int DK = D / 32;        // k-steps of S^T
  __shared__ __attribute__((aligned(16))) uint16_t ks[BKV * KSTR];
  __shared__ __attribute__((aligned(16))) uint16_t vt[D * VSTR];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, quad = lane >> 4;
  const int bh = blockIdx.y;
  const int b = bh / query_heads, h = bh % query_heads;
  const int kvh = h / (query_heads / kv_heads);
  const int q_block = blockIdx.x * 64;
  const int q_wave = q_block + wave * 16;
  const int qi = q_wave + col;           // this lane's query (column of S^T / O^T)
  const int shift = Mk - M;

  const uint16_t* kh = k + (size_t)b * kv_batch_stride + (size_t)kvh * kv_head_stride;
  const uint16_t* vh = v + (size_t)b * kv_batch_stride + (size_t)kvh * kv_head_stride;

  // Q fragments (B operand of S^T): query qi, d = kk*32 + quad*8 + j.
  fa_bf16x8 qf[DK];
  {
    const int qrow = min(qi, M - 1);
    const uint16_t* qp = q + (((size_t)b * query_heads + h) * M + qrow) * D;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) qf[kk] = *reinterpret_cast<const fa_bf16x8*>(qp + kk * 32 + quad * 8);
  }

  fa_f32x4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = fa_f32x4{0.f, 0.f, 0.f, 0.f};
  float run_max = -INFINITY, run_sum = 0.f;

  // Key range this block can see.
  int j_begin = mask ? 0 : key_start;
  int j_end = Mk;
  if (!mask && causal) j_end = min(Mk, q_block + 64 + shift);
  j_begin = max(0, j_begin);
  const int tile_begin = (j_begin / BKV) * BKV;

  for (int j0 = tile_begin; j0 < j_end; j0 += BKV) {
    __syncthreads();
    // Stage K (row-major) and V (transposed) for keys j0 .. j0+63.
    constexpr int VEC = BKV * D / 8;
    for (int idx = threadIdx.x; idx < VEC; idx += 256) {
      const int key = idx / (D / 8), c = idx % (D / 8);
      const int j = j0 + key;
      uint4 kr = make_uint4(0, 0, 0, 0), vr = make_uint4(0, 0, 0, 0);
      if (j < Mk) {
        kr = reinterpret_cast<const uint4*>(kh + (size_t)j * D)[c];
        vr = reinterpret_cast<const uint4*>(vh + (size_t)j * D)[c];
      }
      *reinterpret_cast<uint4*>(ks + key * KSTR + c * 8) = kr;
      const uint32_t raw[4] = {vr.x, vr.y, vr.z, vr.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vt[(c * 8 + 2 * e) * VSTR + key] = (uint16_t)(raw[e] & 0xFFFFu);
        vt[(c * 8 + 2 * e + 1) * VSTR + key] = (uint16_t)(raw[e] >> 16);
      }
    }
    __syncthreads();

    // S^T for 4 sub-tiles of 16 keys.
    float s[4][4];
    float tile_max = -INFINITY;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      fa_f32x4 c4 = fa_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < DK; ++kk) {
        const fa_bf16x8 a = *reinterpret_cast<const fa_bf16x8*>(ks + (st * 16 + col) * KSTR + kk * 32 + quad * 8);
        c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[kk], c4, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = j0 + st * 16 + quad * 4 + i;
        bool keep = j < Mk && qi < M;
        if (keep) {
          if (mask) {
            keep = mask[(size_t)b * mask_batch_stride + (size_t)qi * Mk + j] != 0;
          } else {
            keep = j >= key_start && (!causal || j <= qi + shift);
          }
        }
        const float sc = keep ? c4[i] * scale : -INFINITY;
        s[st][i] = sc;
        tile_max = fmaxf(tile_max, sc);
      }
    }
    tile_max = xor32_max(xor16_max(tile_max));
    const float new_max = fmaxf(run_max, tile_max);
    const float correction = (new_max == -INFINITY) ? 1.f : expf(run_max - new_max);
    float tile_sum = 0.f;
    fa_bf16x4 p[4];
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = (s[st][i] == -INFINITY) ? 0.f : expf(s[st][i] - new_max);
        tile_sum += e;
        p[st][i] = (__bf16)e;
      }
    tile_sum = xor32_sum(xor16_sum(tile_sum));
    run_sum = run_sum * correction + tile_sum;
    run_max = new_max;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      o[t] *= correction;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const fa_bf16x4 a = *reinterpret_cast<const fa_bf16x4*>(vt + (t * 16 + col) * VSTR + st * 16 + quad * 4);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, p[st], o[t], 0, 0, 0);
      }
    }
  }

  if (qi >= M) return;
  const float inv = run_sum > 0.f ? 1.0f / run_sum : 0.f;
  uint16_t* orow = out + ((size_t)b * M + qi) * ((size_t)query_heads * D) + (size_t)h * D;
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    uint2 w;
    w.x = pack_bf16x2(o[t][0] * inv, o[t][1] * inv);
    w.y = pack_bf16x2(o[t][2] * inv, o[t][3] * inv);
    *reinterpret_cast<uint2*>(orow + t * 16 + quad * 4) = w;
  }
}

}  // namespace aoto

#define AOTO_FLASH_INSTANCE(D)                                                                          \
  extern "C" __global__ __launch_bounds__(256) void aoto_flash_attention_d##D(                         \
      const uint16_t* q, const uint16_t* k, const uint16_t* v, long long kv_batch_stride,               \
      long long kv_head_stride, const uint8_t* mask, long long mask_batch_stride, int causal,           \
      int key_start, int M, int Mk, int query_heads, int kv_heads, float scale, uint16_t* out) {        \
    aoto::flash_attention_body<D>(q, k, v, kv_batch_stride, kv_head_stride, mask, mask_batch_stride,    \
                                  causal, key_start, M, Mk, query_heads, kv_heads, scale, out);         \
  }
