// Multi-row direct W4 decode GEMV for the short outputs of a decoder layer at
// batch 1 (q/k/v, gate/up): same semantics and rounding points as w4_gemv.h and
// the streaming form, and the same per-row arithmetic as the streaming form's
// direct instances (chunk order, lane reductions, epilogues).
//
// Why: in the direct streaming form a wave covers 64/LPR rows, and each of its
// lanes loads and normalizes its share of x for every row group. At K = 896
// that is 64 B of x and 64 B of norm weight per 16 B of weights, and the
// normalization costs more VALU time than the dot products. Here a lane keeps
// one normalized copy of its x chunks and applies it to R rows:
//   * a wave covers (64/LPR) row groups x R consecutive rows, one tile, no
//     persistence; the grid is one wave per tile;
//   * x (and the norm weight) are loaded first, then all R x CPL weight chunks,
//     their scales and (bias epilogue) the bias element of the row the lane
//     writes, all as unconditional, clamped loads;
//   * after the R group sums, lane li < R of each row group finishes row li of
//     its group (epilogue and a 2-byte store), so R rows' epilogues run in
//     parallel lanes.
#pragma once

#include "common.h"
#include "w4_gemv_stream.h"

namespace aoto {

// One-wave blocks (tile = block); 64-code scale groups (GS = log2(64 / 32)).
template <int LPR, int CPL, int R, bool NORM, bool PAIRED, bool BIAS>
__device__ void w4_gemv_rows_body(const uint16_t* __restrict__ x, const uint4* __restrict__ words,
                                  const uint16_t* __restrict__ scales, const uint4* __restrict__ up_words,
                                  const uint16_t* __restrict__ up_scales, const uint16_t* __restrict__ norm_w,
                                  float eps, const uint16_t* __restrict__ bias, float alpha, float beta,
                                  uint16_t* __restrict__ y, int K, int N) {
  constexpr int group_shift = 1;
  static_assert(R <= LPR, "a row group's lanes finish its R rows");
  constexpr int RPW = (64 / LPR) * R;  // rows per wave
  const int nchunks = K >> 5;
  const int ngroups = nchunks >> group_shift;
  const int lane = threadIdx.x & 63;
  const int li = lane & (LPR - 1);
  const int tile = blockIdx.x;
  if (tile * RPW >= N) return;  // uniform: the wave has no rows
  const int row0 = tile * RPW + (lane / LPR) * R;

  int cidx[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) cidx[j] = min(li + LPR * j, nchunks - 1);

  DirectActivation<LPR, CPL, NORM> act;
  act.issue(x, norm_w, K, li);
  // x first: loads complete in issue order, so the norm statistic waits for x
  // alone while the weights are still in flight.
  __builtin_amdgcn_sched_barrier(0);
  uint4 q[R][CPL], u[PAIRED ? R : 1][CPL];
  uint16_t s[R][CPL], us[PAIRED ? R : 1][CPL];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int row = min(row0 + i, N - 1);
    const uint4* wrow = words + (size_t)row * nchunks;
    const uint16_t* srow = scales + (size_t)row * ngroups;
#pragma unroll
    for (int j = 0; j < CPL; ++j) q[i][j] = wrow[cidx[j]];
#pragma unroll
    for (int j = 0; j < CPL; ++j) s[i][j] = srow[cidx[j] >> group_shift];
    if (PAIRED) {
      const uint4* urow = up_words + (size_t)row * nchunks;
      const uint16_t* usrow = up_scales + (size_t)row * ngroups;
#pragma unroll
      for (int j = 0; j < CPL; ++j) u[i][j] = urow[cidx[j]];
#pragma unroll
      for (int j = 0; j < CPL; ++j) us[i][j] = usrow[cidx[j] >> group_shift];
    }
  }
  const int out_row = row0 + min(li, R - 1);
  uint32_t bias_bits = 0;
  if (BIAS) bias_bits = bias[min(out_row, N - 1)];

  uint4 xr[CPL][4];
  float cr[CPL];
  act.finish(eps, K, li, xr, cr);

  float total[R], total_up[PAIRED ? R : 1];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float t = 0.f, tu = 0.f;
    // Branch-free over the chunks: a lane past the row's last chunk computes
    // on the clamped chunk and weights it by zero.
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const bool valid = li + LPR * j < nchunks;
      t = fmaf(chunk_dot_fast(q[i][j], xr[j]) - cr[j], valid ? bf16_to_f32(s[i][j]) : 0.f, t);
      if (PAIRED) tu = fmaf(chunk_dot_fast(u[i][j], xr[j]) - cr[j], valid ? bf16_to_f32(us[i][j]) : 0.f, tu);
    }
    total[i] = group_sum<LPR>(t);
    if (PAIRED) total_up[i] = group_sum<LPR>(tu);
  }
  // Lane li < R of the group takes row li's totals.
  float t = total[0], tu = PAIRED ? total_up[0] : 0.f;
#pragma unroll
  for (int i = 1; i < R; ++i) {
    t = li == i ? total[i] : t;
    if (PAIRED) tu = li == i ? total_up[i] : tu;
  }
  if (li < R && out_row < N) {
    float out;
    if (PAIRED) {
      const float g = round_bf16(t);
      out = tu * (g / (1.0f + expf(-g)));
    } else if (BIAS) {
      out = beta * bf16_to_f32(bias_bits) + alpha * t;
    } else {
      out = t;
    }
    y[out_row] = (uint16_t)f32_to_bf16(out);
  }
}

}  // namespace aoto

// aoto_w4_gemv_r{LPR}x{CPL}x{R}_n{NORM}_p{PAIRED}_b{BIAS}: 64-thread blocks, one
// tile each. Argument order: what the first loads need comes first, within the
// 14 preloaded argument dwords (weights, up weights, x, norm weight, shape).
#define AOTO_GEMV_ROWS_INSTANCE(LPR, CPL, R, NORM, PAIRED, BIAS)                                             \
  extern "C" __global__ __launch_bounds__(aoto::kGemvThreads) void                                         \
      aoto_w4_gemv_r##LPR##x##CPL##x##R##_n##NORM##_p##PAIRED##_b##BIAS(                                   \
          const uint4* words, const uint16_t* scales, const uint4* up_words, const uint16_t* up_scales,    \
          const uint16_t* x, const uint16_t* norm_w, int K, int N, const uint16_t* bias, float eps,        \
          float alpha, float beta, uint16_t* y) {                                                         \
    aoto::w4_gemv_rows_body<LPR, CPL, R, NORM, PAIRED, BIAS>(x, words, scales, up_words, up_scales,        \
                                                              norm_w, eps, bias, alpha, beta, y, K, N);    \
  }
// The decoder-layer variants of one lane layout: q/k/v (norm, with or without
// bias), o / down (+residual), plain, and the paired gate/up (norm or not).
#define AOTO_GEMV_ROWS_SHAPE(LPR, CPL, R)              \
  AOTO_GEMV_ROWS_INSTANCE(LPR, CPL, R, 1, 0, 1)        \
  AOTO_GEMV_ROWS_INSTANCE(LPR, CPL, R, 1, 0, 0)        \
  AOTO_GEMV_ROWS_INSTANCE(LPR, CPL, R, 0, 0, 1)        \
  AOTO_GEMV_ROWS_INSTANCE(LPR, CPL, R, 0, 0, 0)        \
  AOTO_GEMV_ROWS_INSTANCE(LPR, CPL, R, 1, 1, 0)        \
  AOTO_GEMV_ROWS_INSTANCE(LPR, CPL, R, 0, 1, 0)
