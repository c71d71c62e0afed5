// Prefill-side pointwise kernels: row RMSNorm, RoPE, and the fused RoPE +
// cache fill that turns the packed q/k/v projection into the attention's head-
// major query and one layer's key/value window.
#pragma once

#include "common.h"

namespace aoto {

// Row RMSNorm (codegen/norm.py:75-323; runtime/mlx_ops/normalization.py:73-119):
//   out[r] = bf16((x[r] * rsqrt(mean(x[r]^2) + eps)) * w), f32 statistics.
// One wave per row, 4 rows per 256-thread block; H % 8 == 0 (16-byte vectors).
// Rows of up to 64 * kRmsVecs vectors (H <= 8192) are held in registers: x and w
// are loaded once, together, so the normalization needs no second round trip.
constexpr int kRmsVecs = 16;
extern "C" __global__ __launch_bounds__(256) void aoto_rms_norm(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ w, float eps,
                                                                uint16_t* __restrict__ out, int rows, int H) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint4* xv = reinterpret_cast<const uint4*>(x + (size_t)row * H);
  const uint4* wv = reinterpret_cast<const uint4*>(w);
  uint4* ov = reinterpret_cast<uint4*>(out + (size_t)row * H);
  const int vecs = H >> 3;
  auto normalized = [&](const uint4 r, const uint4 q, float ns) {
    const uint32_t raw[4] = {r.x, r.y, r.z, r.w};
    const uint32_t wr[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = cvt_pk_bf16((ns * bf16_lo(raw[j])) * bf16_lo(wr[j]), (ns * bf16_hi(raw[j])) * bf16_hi(wr[j]));
    return make_uint4(o[0], o[1], o[2], o[3]);
  };
  auto squares = [](const uint4 r, float ss) {
    const uint32_t raw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = bf16_lo(raw[j]), b = bf16_hi(raw[j]);
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
    return ss;
  };
  float ss = 0.f;
  if (vecs <= 64 * kRmsVecs) {
    uint4 xr[kRmsVecs], wr[kRmsVecs];
#pragma unroll
    for (int i = 0; i < kRmsVecs; ++i) {
      const int c = lane + 64 * i;
      if (c < vecs) {
        xr[i] = xv[c];
        wr[i] = wv[c];
      }
    }
#pragma unroll
    for (int i = 0; i < kRmsVecs; ++i)
      if (lane + 64 * i < vecs) ss = squares(xr[i], ss);
    ss = wave_sum(ss);
    const float ns = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
    for (int i = 0; i < kRmsVecs; ++i) {
      const int c = lane + 64 * i;
      if (c < vecs) ov[c] = normalized(xr[i], wr[i], ns);
    }
    return;
  }
  for (int c = lane; c < vecs; c += 64) ss = squares(xv[c], ss);
  ss = wave_sum(ss);
  const float ns = 1.0f / sqrtf(ss / (float)H + eps);
  for (int c = lane; c < vecs; c += 64) ov[c] = normalized(xv[c], wv[c], ns);
}

// Standalone RoPE over [rows][D] head rows (runtime/mlx_ops/__init__.py:276-280):
// row r uses table row positions[r / rows_per_position] (int64 on the device),
// out = bf16(x * cos + rotate_half(x) * sin). One thread per element.
extern "C" __global__ __launch_bounds__(256) void aoto_rope(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ cos_table,
                                                            const uint16_t* __restrict__ sin_table,
                                                            const long long* __restrict__ positions,
                                                            int rows_per_position, int position_period,
                                                            uint16_t* __restrict__ out, long long rows, int D) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= rows * D) return;
  const long long r = t / D;
  const int d = (int)(t % D);
  const int half = D >> 1;
  const long long p = positions[(r / rows_per_position) % position_period];
  const uint16_t* head = x + (size_t)r * D;
  const float xv = bf16_to_f32(head[d]);
  const float partner = d < half ? -bf16_to_f32(head[d + half]) : bf16_to_f32(head[d - half]);
  const float v = xv * bf16_to_f32(cos_table[(size_t)p * D + d]) + partner * bf16_to_f32(sin_table[(size_t)p * D + d]);
  out[t] = (uint16_t)f32_to_bf16(v);
}

// Fused prefill RoPE + cache fill for one layer. Input: the q/k/v projection
// rows qkv[B][M][W] (q at 0, k at Hq*D, v at (Hq+Hkv)*D). Output:
//   q_out[B][Hq][M][D]      rotated queries, head-major for the attention;
//   pair[0][b][h][slot0+m]  rotated keys, pair[1][b][h][slot0+m] values, in a
//                           [2][B][Hkv][cap][D] window; slots [0, slot0) are
//                           zero-filled when zero_prefix != 0 (the reference's
//                           left pad of the compact cache, models/decoder.py:870-887).
// positions[b*M + m] (int64, device) picks the table row of token m.
extern "C" __global__ __launch_bounds__(256) void aoto_rope_qkv_prefill(
    const uint16_t* __restrict__ qkv, const long long* __restrict__ positions,
    const uint16_t* __restrict__ cos_table, const uint16_t* __restrict__ sin_table, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ pair, int batch, int M, int query_heads, int kv_heads, int D, int cap, int slot0,
    int zero_prefix) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const int half = D >> 1;
  const int W = (query_heads + 2 * kv_heads) * D;
  const long long q_items = (long long)batch * query_heads * M * D;
  const long long k_items = (long long)batch * kv_heads * M * D;
  const size_t head_stride = (size_t)cap * D;
  const size_t pair_stride = (size_t)batch * kv_heads * head_stride;
  if (t < q_items + 2 * k_items) {
    const bool is_q = t < q_items;
    long long u = is_q ? t : t - q_items;
    const bool is_v = !is_q && u >= k_items;
    if (is_v) u -= k_items;
    const int heads = is_q ? query_heads : kv_heads;
    const int d = (int)(u % D);
    const int m = (int)((u / D) % M);
    const long long bh = u / ((long long)D * M);
    const int b = (int)(bh / heads), h = (int)(bh % heads);
    const int col0 = is_q ? h * D : (is_v ? (query_heads + kv_heads + h) * D : (query_heads + h) * D);
    const uint16_t* head = qkv + ((size_t)b * M + m) * W + col0;
    if (is_v) {
      pair[pair_stride + ((size_t)b * kv_heads + h) * head_stride + (size_t)(slot0 + m) * D + d] = head[d];
      return;
    }
    const long long p = positions[(size_t)b * M + m];
    const float x = bf16_to_f32(head[d]);
    const float partner = d < half ? -bf16_to_f32(head[d + half]) : bf16_to_f32(head[d - half]);
    const float v = x * bf16_to_f32(cos_table[(size_t)p * D + d]) + partner * bf16_to_f32(sin_table[(size_t)p * D + d]);
    const uint16_t bits = (uint16_t)f32_to_bf16(v);
    if (is_q) {
      q_out[(((size_t)b * query_heads + h) * M + m) * D + d] = bits;
    } else {
      pair[((size_t)b * kv_heads + h) * head_stride + (size_t)(slot0 + m) * D + d] = bits;
    }
    return;
  }
  if (!zero_prefix) return;
  const long long z = t - (q_items + 2 * k_items);
  const long long prefix = (long long)slot0 * D;
  if (z >= 2LL * batch * kv_heads * prefix) return;
  const long long hh = z / prefix;
  pair[(size_t)hh * head_stride + (size_t)(z % prefix)] = 0;
}

}  // namespace aoto
