// Prefill W4 GEMM on bf16 MFMA with the dequant fused in registers.
//
//   Y[m][n] = epilogue( sum_k X[m][k] * bf16(code[n][k] * s[n][k/group]) )
//
// The reference prefill unpacks the weight to bf16 (codegen/quantize.py:27-63,
// models/quantized.py:61-76) and runs a tiled GEMM over it with a bias /
// residual / silu_mul epilogue (codegen/matmul.py:1443-1471, 1721-1742). Here
// the unpacked weight never exists in memory: each packed int32 word is exactly
// one lane's 8-element operand of v_mfma_f32_16x16x32_bf16 (8 consecutive k of
// one row), so lanes load words straight from HBM and expand them in registers
// to the same bf16(code * scale) values.
//
// MFMA formulation: C^T = W . X^T per 16x16 tile, so
//   A (16 n x 32 k): lane l holds W[n0 + l%16][k0 + (l/16)*8 + j]  -> one packed word
//   B (32 k x 16 m): lane l holds X[m0 + l%16][k0 + (l/16)*8 + j]  -> 16 B of an X row
//   C (16 n x 16 m): lane l holds Y[m0 + l%16][n0 + (l/16)*4 + i]  -> 8-byte stores
//
// Block: 4 waves side by side along n; wave tile TN x TM 16x16 tiles
// (block tile BN = 64*TN columns by BM = 16*TM rows). The X tile [BM][64] is
// staged in LDS (rows padded by 16 B) and shared by the four waves; each wave
// dequantizes only its own words, once, and reuses them for all TM row tiles
// (TM = 8 keeps the dequant VALU work under the MFMA time).
//
// The eight-bit form (BITS = 8, the reference's quantize_bits=8 weights: four
// codes per int32 word, byte k of word j = code 4j+k) is the same kernel with
// two words (one 8-byte load) per lane operand instead of one.
#pragma once

#include <utility>

#include "common.h"
#include "gemm_args.h"

namespace aoto {

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));

// Eight bf16(code * s) values of one packed word, in k order.
AOTO_DEVICE bf16x8_v dequant_word(uint32_t w, float s) {
  bf16x8_v out;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int code = (int)(w << (28 - 4 * j)) >> 28;
    out[j] = (__bf16)((float)code * s);
  }
  return out;
}

// Eight bf16(code * s) values of two eight-bit words (bytes 0..3 of lo, then hi).
AOTO_DEVICE bf16x8_v dequant_word(uint2 w, float s) {
  bf16x8_v out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    out[j] = (__bf16)((float)((int)(w.x << (24 - 8 * j)) >> 24) * s);
    out[4 + j] = (__bf16)((float)((int)(w.y << (24 - 8 * j)) >> 24) * s);
  }
  return out;
}

// The unit of packed weight that holds one lane's 8 consecutive codes.
template <int BITS> struct GemmWord;
template <> struct GemmWord<4> { using type = uint32_t; };
template <> struct GemmWord<8> { using type = uint2; };

constexpr int kGemmBK = 128;                 // k per step: 16 packed words of a weight row
constexpr int kGemmLdsStride = kGemmBK + 8;  // bf16 per staged X row

// k-steps whose loads are in flight: one step ahead for every tile. Measured on
// MI355X for the 64-row tiles at M = 128 (Qwen2-0.5B q/k/v, o, gate/up, down):
// 8.17 / 7.54 / 11.78 / 11.47 us with 2 slots, 8.41 / 7.78 / 12.19 / 11.75 with
// 3, 8.63 / 7.98 / 13.33 / 12.69 with 4 - a 128-k step's loads are enough to
// cover, and more slots only cost registers.
constexpr int gemm_depth(int) { return 2; }

// f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>) in order: the
// step index is a constant in each call, so register arrays indexed by it stay
// in registers whatever the unroller decides.
template <int... I, class F>
AOTO_DEVICE void static_for_impl(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
AOTO_DEVICE void static_for(F&& f) {
  static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

// RoPE and the cache fill of one staged q/k/v block: BM rows of the projection
// from m0, BN columns - whole heads - from n0, as bf16 in tile[r][c] (row
// stride TS). Item i = r * BN/8 + c8 of a thread's IPT = BM*BN/2048 items is one
// (token, head, 4 consecutive d of the head's first half) with its partner
// columns d + D/2, the same arithmetic as aoto_rope_qkv_prefill: v = x cos +
// partner sin from the rounded projection, one rounding; values are copied
// unrotated. The table rows of each item are loaded by RopeRows (early, so the
// epilogue does not wait for them). Block row 0 also zeroes the prefix slots
// of the block's key and value heads when asked.
template <int BM, int BN>
struct RopeRows {
  static constexpr int IPT = BM * BN / 2048;
  long long pos[IPT];
  uint2 cs[IPT][4];  // cos[d..d+4), cos[d+D/2..), sin[d..), sin[d+D/2..)

  AOTO_DEVICE static int row_of(int j) { return ((int)threadIdx.x + 256 * j) / (BN / 8); }
  AOTO_DEVICE static int col_of(int j, int D) {  // first-half column of the item within the block
    const int c8 = ((int)threadIdx.x + 256 * j) % (BN / 8), quads = D / 8;
    return (c8 / quads) * D + 4 * (c8 % quads);
  }
  AOTO_DEVICE void load_positions(const QkvRope& r, int M, int m0) {
#pragma unroll
    for (int j = 0; j < IPT; ++j) pos[j] = r.positions[min(m0 + row_of(j), M - 1)];
  }
  AOTO_DEVICE void load_tables(const QkvRope& r) {
    const int D = r.head_dim, half = D >> 1;
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int d = col_of(j, D) % D;
      const uint16_t* cr = r.cos_table + (size_t)pos[j] * D + d;
      const uint16_t* sr = r.sin_table + (size_t)pos[j] * D + d;
      cs[j][0] = *reinterpret_cast<const uint2*>(cr);
      cs[j][1] = *reinterpret_cast<const uint2*>(cr + half);
      cs[j][2] = *reinterpret_cast<const uint2*>(sr);
      cs[j][3] = *reinterpret_cast<const uint2*>(sr + half);
    }
  }
};

template <int BM, int BN, int TS>
AOTO_DEVICE void rope_tile(const uint16_t* tile, const RopeRows<BM, BN>& rows, const QkvRope& r, int M, int m0,
                           int n0) {
  const int D = r.head_dim, half = D >> 1;
  const int h0 = n0 / D;
  const size_t head_stride = (size_t)r.cap * D;
  const size_t pair_stride = (size_t)r.kv_heads * head_stride;
#pragma unroll
  for (int j = 0; j < RopeRows<BM, BN>::IPT; ++j) {
    const int row = RopeRows<BM, BN>::row_of(j);
    const int m = m0 + row;
    if (m >= M) continue;
    const int c = RopeRows<BM, BN>::col_of(j, D);
    const int h = h0 + c / D, d = c % D;
    const uint2 ya = *reinterpret_cast<const uint2*>(tile + row * TS + c);
    const uint2 yb = *reinterpret_cast<const uint2*>(tile + row * TS + c + half);
    uint16_t* dst;
    if (h < r.query_heads)
      dst = r.q_out + ((size_t)h * M + m) * D;
    else if (h < r.query_heads + r.kv_heads)
      dst = r.pair + (size_t)(h - r.query_heads) * head_stride + (size_t)(r.slot0 + m) * D;
    else
      dst = r.pair + pair_stride + (size_t)(h - r.query_heads - r.kv_heads) * head_stride + (size_t)(r.slot0 + m) * D;
    if (h >= r.query_heads + r.kv_heads) {
      *reinterpret_cast<uint2*>(dst + d) = ya;
      *reinterpret_cast<uint2*>(dst + d + half) = yb;
      continue;
    }
    const float xa[4] = {bf16_lo(ya.x), bf16_hi(ya.x), bf16_lo(ya.y), bf16_hi(ya.y)};
    const float xb[4] = {bf16_lo(yb.x), bf16_hi(yb.x), bf16_lo(yb.y), bf16_hi(yb.y)};
    const uint2 ca = rows.cs[j][0], cb = rows.cs[j][1], sa = rows.cs[j][2], sb = rows.cs[j][3];
    const float c0[4] = {bf16_lo(ca.x), bf16_hi(ca.x), bf16_lo(ca.y), bf16_hi(ca.y)};
    const float c1[4] = {bf16_lo(cb.x), bf16_hi(cb.x), bf16_lo(cb.y), bf16_hi(cb.y)};
    const float s0[4] = {bf16_lo(sa.x), bf16_hi(sa.x), bf16_lo(sa.y), bf16_hi(sa.y)};
    const float s1[4] = {bf16_lo(sb.x), bf16_hi(sb.x), bf16_lo(sb.y), bf16_hi(sb.y)};
    float ra[4], rb[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      ra[k] = xa[k] * c0[k] + (-xb[k]) * s0[k];  // first half: x cos - x[d + D/2] sin
      rb[k] = xb[k] * c1[k] + xa[k] * s1[k];     // second half: x cos + x[d - D/2] sin
    }
    *reinterpret_cast<uint2*>(dst + d) = make_uint2(pack_bf16x2(ra[0], ra[1]), pack_bf16x2(ra[2], ra[3]));
    *reinterpret_cast<uint2*>(dst + d + half) = make_uint2(pack_bf16x2(rb[0], rb[1]), pack_bf16x2(rb[2], rb[3]));
  }
  if (!r.zero_prefix || blockIdx.y != 0) return;
  const int prefix = r.slot0 * D / 4;  // 8-byte stores per head
  for (int hh = 0; hh < BN / D; ++hh) {
    const int h = h0 + hh;
    if (h < r.query_heads) continue;
    uint16_t* base = r.pair + (size_t)(h - r.query_heads) * head_stride;  // k heads, then v heads
    for (int z = threadIdx.x; z < prefix; z += blockDim.x)
      *reinterpret_cast<uint2*>(base + (size_t)z * 4) = make_uint2(0u, 0u);
  }
}

// Split-K: blockIdx.z selects the reduction slice [z*kslice, min(K, (z+1)*kslice));
// with `partials` non-null the block stores its f32 tile to partials[z][m][n]
// and aoto_w4_gemm_reduce applies the sum and the epilogue.
// PAIRED: the MLP's gate and up projections in one pass (the decode path's
// paired GEMV, at M > 1): the block also holds the up weight's words for the
// same columns, accumulates both against the one staged X tile and stores
// bf16(up * silu(bf16(gate))) - the values the gate GEMM followed by the up
// GEMM with the gate epilogue produce, with one launch and one read of X.
// Split partials are gate at partials[z], up at partials[splits + z]
// (aoto_w4_gemm_reduce_paired).
//
// k order within a step: the 128 k of a step are 16 eight-code units; lane
// quad q holds units 4q .. 4q+3 of its weight row (one 16-byte load for 4-bit
// codes, one scale: 32 aligned k never straddle a group) and the j-th product
// of the step takes unit 4q + j from every lane - for both operands, so the
// sum over k is the same, only its order differs. A step past K (K = 64 mod
// 128) zeroes the codes of quads 2 and 3.
//
// ROPE (unsplit q/k/v, block columns a whole number of heads): the epilogue
// also stages the block's bf16 tile in LDS and applies RoPE and the cache fill
// to it (aoto_rope_qkv_prefill on the tile's heads, same values), so the
// projection, its bias, RoPE and the cache fill are one launch.
template <int BITS, int TN, int TM, int DEPTH, bool BIAS, bool RESIDUAL, bool GATE, bool PAIRED = false,
          bool ROPE = false>
__device__ void w4_gemm_body(const uint16_t* __restrict__ X, const typename GemmWord<BITS>::type* __restrict__ words,
                             const uint16_t* __restrict__ scales, const uint16_t* __restrict__ bias,
                             const uint16_t* __restrict__ residual, const uint16_t* __restrict__ gate,
                             uint16_t* __restrict__ Y, int M, int N, int K, int group, int kslice,
                             float* __restrict__ partials,
                             const typename GemmWord<BITS>::type* __restrict__ up_words = nullptr,
                             const uint16_t* __restrict__ up_scales = nullptr, const QkvRope rope = QkvRope{}) {
  static_assert(!(PAIRED && (BIAS || RESIDUAL || GATE)), "the paired form has its own epilogue");
  static_assert(!(ROPE && (PAIRED || RESIDUAL || GATE)), "RoPE follows the bias epilogue only");
  constexpr int BM = 16 * TM;
  constexpr int BN = 64 * TN;
  constexpr int XVEC = BM * (kGemmBK / 8);        // 16-byte vectors per X tile
  constexpr int XPT = (XVEC + 255) / 256;         // per thread
  constexpr int NP = PAIRED ? 2 : 1;              // weight matrices: gate (or the only one), up
  constexpr int WV = BITS / 4;                    // 16-byte vectors per lane's 4 units
  __shared__ __attribute__((aligned(16))) uint16_t xs[2 * BM * kGemmLdsStride];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_block = blockIdx.x * BN;
  const int m_block = blockIdx.y * BM;
  const int n_wave = n_block + wave * (16 * TN);
  using Word = typename GemmWord<BITS>::type;
  const int kw = K >> 3;           // 8-code units per weight row
  const int groups = K / group;
  const float inv_g32 = 32.0f / (float)group;  // 32-k chunks -> group: exact for the chunk counts here
  const int col = lane & 15;       // n (A) / m (B, C) within a tile
  const int quad = lane >> 4;      // unit block of 4 (A, B) / n block of 4 (C)

  f32x4_v acc[NP][TN][TM];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int u = 0; u < TM; ++u) acc[p][t][u] = f32x4_v{0.f, 0.f, 0.f, 0.f};

  // Rows of W this lane reads (clamped: rows past N compute garbage that is never stored).
  int wrow[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t) wrow[t] = min(n_wave + t * 16 + col, N - 1);

  // DEPTH slots of loads in flight: every load is unconditional (a step past the
  // block's slice re-reads its last step, a cache hit), so the wait for a slot
  // is an exact count of the loads issued after it. Native vector types: a HIP
  // uint4 struct copied from global memory lowers to a memcpy through a stack slot.
  typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));
  u32x4_v xr[DEPTH][XPT];
  u32x4_v wr[DEPTH][NP][TN][WV];
  uint16_t sr[DEPTH][NP][TN];
  auto load = [&](auto slot_c, int k0) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
#pragma unroll
    for (int v = 0; v < XPT; ++v) {
      const int idx = min((int)threadIdx.x + v * 256, XVEC - 1);
      const int r = idx / (kGemmBK / 8), c = idx % (kGemmBK / 8);
      const int m = min(m_block + r, M - 1);  // rows past M feed outputs that are never stored
      int k = k0 + c * 8;
      k = k < K ? k : k - kGemmBK / 2;         // the half step's upper half: any finite X (codes are 0)
      xr[slot][v] = *reinterpret_cast<const u32x4_v*>(X + (size_t)m * K + k);
    }
    const int ku = (k0 >> 3) + 4 * quad;      // this lane's first unit
    const int kuc = ku < kw ? ku : ku - 8;    // (half step: in-bounds, zeroed below)
    const int sidx = (int)(((float)(ku >> 2) + 0.5f) * inv_g32);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const Word* wm = p == 0 ? words : up_words;
      const uint16_t* sm = p == 0 ? scales : up_scales;
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const u32x4_v* src = reinterpret_cast<const u32x4_v*>(wm + (size_t)wrow[t] * kw + kuc);
#pragma unroll
        for (int e = 0; e < WV; ++e) wr[slot][p][t][e] = src[e];
        sr[slot][p][t] = sm[(size_t)wrow[t] * groups + min(sidx, groups - 1)];
      }
    }
  };
  auto store_x = [&](auto slot_c, uint16_t* buf) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
#pragma unroll
    for (int v = 0; v < XPT; ++v) {
      const int idx = threadIdx.x + v * 256;
      if (idx < XVEC) {
        const int r = idx / (kGemmBK / 8), c = idx % (kGemmBK / 8);
        *reinterpret_cast<u32x4_v*>(buf + r * kGemmLdsStride + c * 8) = xr[slot][v];
      }
    }
  };

  // ROPE: the block's table rows are loaded early - positions now, the cos/sin
  // rows after the first step (small blocks) or ahead of the epilogue (blocks
  // whose rows would not fit the loop's registers) - so the RoPE tail does not
  // wait on two dependent memory round trips.
  constexpr bool EARLY_TABLES = BM * BN <= 4096;
  RopeRows<BM, BN> rope_rows;
  if constexpr (ROPE) rope_rows.load_positions(rope, M, m_block);
  // the bias of this lane's columns, loaded before the loop rather than in the epilogue
  uint2 bias_cols[TN];
  if constexpr (BIAS) {
#pragma unroll
    for (int t = 0; t < TN; ++t)
      bias_cols[t] = *reinterpret_cast<const uint2*>(bias + min(n_wave + t * 16 + quad * 4, N - 4));
  }

  const int kb = blockIdx.z * kslice;
  const int ke = min(K, kb + kslice);
  const int steps = (ke - kb + kGemmBK - 1) / kGemmBK;
  // The loop starts DEPTH - 1 steps early with the compute skipped, so every
  // slot is loaded inside the loop: with a separate prologue the registers it
  // loads and the ones the loop carries differ, and the wait count at the loop
  // head falls back to the prologue's latest load (one step of prefetch).
  // s0 = 1 - DEPTH (mod DEPTH): sub-step d loads step s0 + d + DEPTH - 1 into
  // slot d and computes step s0 + d from slot (d + 1) % DEPTH. X tiles are
  // double-buffered in LDS: one barrier per step orders the store of step s
  // before its reads and the reads of step s - 2 before the store that reuses
  // their buffer.
  for (int s0 = 1 - DEPTH; s0 < steps; s0 += DEPTH) {
    static_for<DEPTH>([&](auto d_c) __attribute__((always_inline)) {
      constexpr int d = decltype(d_c)::value;
      constexpr int cs = (d + 1) % DEPTH;
      const int s = s0 + d;
      load(d_c, kb + min(s + DEPTH - 1, steps - 1) * kGemmBK);
      if (s >= 0 && s < steps) {
        uint16_t* buf = xs + (s & 1) * (BM * kGemmLdsStride);
        store_x(std::integral_constant<int, cs>{}, buf);
        // this lane's units past K (the half step) contribute zero codes
        const bool live = kb + s * kGemmBK + 32 * quad < ke;
        float scur[NP][TN];
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int t = 0; t < TN; ++t) scur[p][t] = bf16_to_f32(sr[cs][p][t]);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // all TM operands read before the products (one LDS round trip, not TM)
          bf16x8_v b[TM];
#pragma unroll
          for (int u = 0; u < TM; ++u)
            b[u] = *reinterpret_cast<const bf16x8_v*>(buf + (u * 16 + col) * kGemmLdsStride + (4 * quad + j) * 8);
          bf16x8_v a[NP][TN];
#pragma unroll
          for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int t = 0; t < TN; ++t) {
              Word w;
              if constexpr (BITS == 4) {
                w = live ? wr[cs][p][t][0][j] : 0u;
              } else {
                const u32x4_v& h = wr[cs][p][t][j >> 1];
                w = live ? make_uint2(h[(j & 1) * 2], h[(j & 1) * 2 + 1]) : make_uint2(0u, 0u);
              }
              a[p][t] = dequant_word(w, scur[p][t]);
            }
#pragma unroll
          for (int u = 0; u < TM; ++u)
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
              for (int t = 0; t < TN; ++t)
                acc[p][t][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[p][t], b[u], acc[p][t][u], 0, 0, 0);
        }
        if constexpr (ROPE && EARLY_TABLES)
          if (s == 0) rope_rows.load_tables(rope);
      }
    });
  }

  if (partials != nullptr) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float* part = partials + ((size_t)p * gridDim.z + blockIdx.z) * M * N;
#pragma unroll
      for (int u = 0; u < TM; ++u) {
        const int m = m_block + u * 16 + col;
        if (m >= M) continue;
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          const int n = n_wave + t * 16 + quad * 4;
          if (n >= N) continue;
          *reinterpret_cast<float4*>(part + (size_t)m * N + n) =
              make_float4(acc[p][t][u][0], acc[p][t][u][1], acc[p][t][u][2], acc[p][t][u][3]);
        }
      }
    }
    return;
  }
  // Epilogue: lane holds Y[m0 + col][n0 + quad*4 + i].
  constexpr int YS = BN + 8;  // ROPE: bf16 per staged tile row
  static_assert(!ROPE || BM * YS <= 2 * BM * kGemmLdsStride, "the staged tile fits the X tiles");
  if constexpr (ROPE) {
    if constexpr (!EARLY_TABLES) rope_rows.load_tables(rope);
    __syncthreads();  // every wave is past its last read of the X tiles
  }
#pragma unroll
  for (int u = 0; u < TM; ++u) {
    const int m = m_block + u * 16 + col;
    if (m >= M) continue;
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const int n = n_wave + t * 16 + quad * 4;
      if (n >= N) continue;
      float v[4] = {acc[0][t][u][0], acc[0][t][u][1], acc[0][t][u][2], acc[0][t][u][3]};
      if (PAIRED) {
        // gate rounded to bf16 as the gate GEMM stores it, then the up epilogue
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float g = round_bf16(v[i]);
          v[i] = acc[1][t][u][i] * (g / (1.0f + expf(-g)));
        }
      }
      if (BIAS) {
        const uint2 bb = bias_cols[t];
        v[0] += bf16_lo(bb.x);
        v[1] += bf16_hi(bb.x);
        v[2] += bf16_lo(bb.y);
        v[3] += bf16_hi(bb.y);
      }
      if (RESIDUAL) {
        const uint2 rr = *reinterpret_cast<const uint2*>(residual + (size_t)m * N + n);
        v[0] += bf16_lo(rr.x);
        v[1] += bf16_hi(rr.x);
        v[2] += bf16_lo(rr.y);
        v[3] += bf16_hi(rr.y);
      }
      if (GATE) {
        const uint2 gg = *reinterpret_cast<const uint2*>(gate + (size_t)m * N + n);
        const float g[4] = {bf16_lo(gg.x), bf16_hi(gg.x), bf16_lo(gg.y), bf16_hi(gg.y)};
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = v[i] * (g[i] / (1.0f + expf(-g[i])));
      }
      uint2 o;
      o.x = pack_bf16x2(v[0], v[1]);
      o.y = pack_bf16x2(v[2], v[3]);
      *reinterpret_cast<uint2*>(Y + (size_t)m * N + n) = o;
      if (ROPE) *reinterpret_cast<uint2*>(xs + (u * 16 + col) * YS + (n - n_block)) = o;
    }
  }
  if constexpr (ROPE) {
    __syncthreads();
    rope_tile<BM, BN, YS>(xs, rope_rows, rope, M, m_block, n_block);
  }
}

// v += partials[s][e .. e+4) for s = 0 .. splits-1, added in split order; the
// loads are issued eight splits at a time (a loop that waits for each split's
// load costs a memory round trip per split).
AOTO_DEVICE void sum_partials(const float* __restrict__ partials, int splits, size_t stride, size_t e,
                              float (&v)[4]) {
  int s = 0;
  for (; s + 8 <= splits; s += 8) {
    float4 p[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) p[u] = *reinterpret_cast<const float4*>(partials + (size_t)(s + u) * stride + e);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      v[0] += p[u].x;
      v[1] += p[u].y;
      v[2] += p[u].z;
      v[3] += p[u].w;
    }
  }
  float4 p[8];
#pragma unroll
  for (int u = 0; u < 8; ++u)
    if (s + u < splits) p[u] = *reinterpret_cast<const float4*>(partials + (size_t)(s + u) * stride + e);
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    if (s + u < splits) {
      v[0] += p[u].x;
      v[1] += p[u].y;
      v[2] += p[u].z;
      v[3] += p[u].w;
    }
  }
}

// v[0..8) += partials[s][e .. e+8) in split order (per element the same adds as
// sum_partials on each half), four splits' loads in flight at a time.
AOTO_DEVICE void sum_partials8(const float* __restrict__ partials, int splits, size_t stride, size_t e,
                               float (&v)[8]) {
  for (int s = 0; s < splits; s += 4) {
    float4 p[4][2];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (s + u < splits) {
        const float4* src = reinterpret_cast<const float4*>(partials + (size_t)(s + u) * stride + e);
        p[u][0] = src[0];
        p[u][1] = src[1];
      }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (s + u < splits) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          v[4 * h] += p[u][h].x;
          v[4 * h + 1] += p[u][h].y;
          v[4 * h + 2] += p[u][h].z;
          v[4 * h + 3] += p[u][h].w;
        }
      }
  }
}

// Sum the split-K partial tiles and apply the epilogue: one thread per 4 outputs.
// (The f32 sum of the slices replaces the single-block accumulation; each slice
// is itself an f32 MFMA accumulation, so only the summation order differs.)
extern "C" __global__ __launch_bounds__(256) void aoto_w4_gemm_reduce(
    const float* __restrict__ partials, int splits, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ residual, const uint16_t* __restrict__ gate, uint16_t* __restrict__ Y, int M,
    int N) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long quads = (long long)M * N / 4;
  if (t >= quads) return;
  const size_t e = (size_t)t * 4;
  const int n = (int)(e % N);
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  sum_partials(partials, splits, (size_t)M * N, e, v);
  if (bias != nullptr) {
    const uint2 bb = *reinterpret_cast<const uint2*>(bias + n);
    v[0] += bf16_lo(bb.x);
    v[1] += bf16_hi(bb.x);
    v[2] += bf16_lo(bb.y);
    v[3] += bf16_hi(bb.y);
  }
  if (residual != nullptr) {
    const uint2 rr = *reinterpret_cast<const uint2*>(residual + e);
    v[0] += bf16_lo(rr.x);
    v[1] += bf16_hi(rr.x);
    v[2] += bf16_lo(rr.y);
    v[3] += bf16_hi(rr.y);
  }
  if (gate != nullptr) {
    const uint2 gg = *reinterpret_cast<const uint2*>(gate + e);
    const float g[4] = {bf16_lo(gg.x), bf16_hi(gg.x), bf16_lo(gg.y), bf16_hi(gg.y)};
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = v[i] * (g[i] / (1.0f + expf(-g[i])));
  }
  uint2 o;
  o.x = pack_bf16x2(v[0], v[1]);
  o.y = pack_bf16x2(v[2], v[3]);
  *reinterpret_cast<uint2*>(Y + e) = o;
}


// The split-K sum with a residual epilogue followed by the row RMSNorm of its
// result (the decoder layer's o and down projections, each followed by the next
// block's norm): one block per row, one 8-wide vector of the row per thread
// (two for rows over 2048), its partial loads issued together:
//   y[m]    = bf16(residual[m] + sum of partials[..][m])      (aoto_w4_gemm_reduce)
//   norm[m] = bf16((ns * y[m][e]) * w[e]),  ns = 1 / sqrt(mean(y[m]^2) + eps)
// y equals the reduce launch's bit for bit; the sum of squares is a block sum,
// so ns may differ from aoto_rms_norm's wave-serial sum in the last f32 bits.
// y may alias residual.
extern "C" __global__ __launch_bounds__(256) void aoto_w4_gemm_reduce_norm(
    const float* __restrict__ partials, int splits, const uint16_t* residual, uint16_t* Y,
    const uint16_t* __restrict__ norm_w, float eps, uint16_t* __restrict__ norm_out, int M, int N) {
  __shared__ float scratch[4];
  const int row = blockIdx.x;
  const int vecs = N >> 3;
  uint32_t yv[2][4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c >= vecs) continue;
    const size_t e = (size_t)row * N + (size_t)c * 8;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    sum_partials8(partials, splits, (size_t)M * N, e, v);
    if (residual != nullptr) {
      const uint4 rr = *reinterpret_cast<const uint4*>(residual + e);
      const uint32_t r[4] = {rr.x, rr.y, rr.z, rr.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] += bf16_lo(r[j]);
        v[2 * j + 1] += bf16_hi(r[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      yv[i][j] = pack_bf16x2(v[2 * j], v[2 * j + 1]);
      const float a = bf16_lo(yv[i][j]), b = bf16_hi(yv[i][j]);
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
    *reinterpret_cast<uint4*>(Y + e) = make_uint4(yv[i][0], yv[i][1], yv[i][2], yv[i][3]);
  }
  ss = block_sum<256>(ss, scratch);
  const float ns = 1.0f / sqrtf(ss / (float)N + eps);
  const uint4* wv = reinterpret_cast<const uint4*>(norm_w);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c >= vecs) continue;
    const uint4 q = wv[c];
    const uint32_t wr[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = cvt_pk_bf16((ns * bf16_lo(yv[i][j])) * bf16_lo(wr[j]), (ns * bf16_hi(yv[i][j])) * bf16_hi(wr[j]));
    *reinterpret_cast<uint4*>(norm_out + (size_t)row * N + (size_t)c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// The RoPE / cache-fill tail of aoto_w4_gemm_reduce_rope and aoto_rope_qkv_rows for
// one thread's quad: the bf16 projection values ya (d .. d+3 of head h, token m) and
// yb (the partner columns d + D/2 ..); RoPE in f32 from the rounded pair, one rounding.
AOTO_DEVICE void rope_quad_store(uint2 ya, uint2 yb, int m, int h, int d, int M,
                                 const long long* __restrict__ positions, const uint16_t* __restrict__ cos_table,
                                 const uint16_t* __restrict__ sin_table, uint16_t* __restrict__ q_out,
                                 uint16_t* __restrict__ pair, int query_heads, int kv_heads, int D, int cap,
                                 int slot0) {
  const int half = D >> 1;
  const size_t head_stride = (size_t)cap * D;
  const size_t pair_stride = (size_t)kv_heads * head_stride;
  uint16_t* dst;
  if (h < query_heads)
    dst = q_out + ((size_t)h * M + m) * D;
  else if (h < query_heads + kv_heads)
    dst = pair + (size_t)(h - query_heads) * head_stride + (size_t)(slot0 + m) * D;
  else
    dst = pair + pair_stride + (size_t)(h - query_heads - kv_heads) * head_stride + (size_t)(slot0 + m) * D;
  if (h >= query_heads + kv_heads) {  // values: the stored projection, unrotated
    *reinterpret_cast<uint2*>(dst + d) = ya;
    *reinterpret_cast<uint2*>(dst + d + half) = yb;
    return;
  }
  const float xa[4] = {bf16_lo(ya.x), bf16_hi(ya.x), bf16_lo(ya.y), bf16_hi(ya.y)};
  const float xb[4] = {bf16_lo(yb.x), bf16_hi(yb.x), bf16_lo(yb.y), bf16_hi(yb.y)};
  const long long p = positions[m];
  const uint16_t* cr = cos_table + (size_t)p * D;
  const uint16_t* sr = sin_table + (size_t)p * D;
  const uint2 ca = *reinterpret_cast<const uint2*>(cr + d), cb = *reinterpret_cast<const uint2*>(cr + d + half);
  const uint2 sa = *reinterpret_cast<const uint2*>(sr + d), sb = *reinterpret_cast<const uint2*>(sr + d + half);
  const float c0[4] = {bf16_lo(ca.x), bf16_hi(ca.x), bf16_lo(ca.y), bf16_hi(ca.y)};
  const float c1[4] = {bf16_lo(cb.x), bf16_hi(cb.x), bf16_lo(cb.y), bf16_hi(cb.y)};
  const float s0[4] = {bf16_lo(sa.x), bf16_hi(sa.x), bf16_lo(sa.y), bf16_hi(sa.y)};
  const float s1[4] = {bf16_lo(sb.x), bf16_hi(sb.x), bf16_lo(sb.y), bf16_hi(sb.y)};
  float ra[4], rb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ra[i] = xa[i] * c0[i] + (-xb[i]) * s0[i];  // first half: x cos - x[d + D/2] sin
    rb[i] = xb[i] * c1[i] + xa[i] * s1[i];     // second half: x cos + x[d - D/2] sin
  }
  *reinterpret_cast<uint2*>(dst + d) = make_uint2(pack_bf16x2(ra[0], ra[1]), pack_bf16x2(ra[2], ra[3]));
  *reinterpret_cast<uint2*>(dst + d + half) = make_uint2(pack_bf16x2(rb[0], rb[1]), pack_bf16x2(rb[2], rb[3]));
}

// Zero-fill of the cache window's slots [0, slot0) for zero_prefix: thread z of
// 2 Hkv slot0 D / 4 stores one 8-byte zero (threads past the range do nothing).
AOTO_DEVICE void rope_zero_prefix(long long z, uint16_t* __restrict__ pair, int kv_heads, int D, int cap,
                                  int slot0) {
  const long long prefix = (long long)slot0 * D / 4;
  if (z >= 2LL * kv_heads * prefix) return;
  const long long hh = z / prefix;
  *reinterpret_cast<uint2*>(pair + (size_t)hh * cap * D + (size_t)(z % prefix) * 4) = make_uint2(0u, 0u);
}

// The packed q/k/v projection's split-K sum fused with its bias, the bf16 value
// the projection stores, RoPE and the layer's cache fill: aoto_w4_gemm_reduce (bias
// epilogue) followed by aoto_rope_qkv_prefill in one launch, with the same values
// (the rounding of y, then RoPE in f32 from the rounded pair, one rounding).
// Input partials[s][m][W] (W = (Hq + 2 Hkv) D, q at 0, k at Hq D, v after); one
// thread per (token m, head, 4 consecutive d of the head's first half) and the
// partner columns d + D/2, so the rotation needs no exchange. Writes
//   y[m][W]                   the projection (what aoto_w4_gemm_reduce stores);
//   q_out[h][m][D]            rotated queries, head-major;
//   pair[0][h][slot0 + m][D]  rotated keys, pair[1][h][slot0 + m][D] values, of a
//                             [2][Hkv][cap][D] window; with zero_prefix, slots
//                             [0, slot0) of both are zeroed (batch 1).
// positions[m] (int64) picks the table row of token m.
extern "C" __global__ __launch_bounds__(256) void aoto_w4_gemm_reduce_rope(
    const float* __restrict__ partials, int splits, const uint16_t* __restrict__ bias, uint16_t* __restrict__ Y,
    int M, const long long* __restrict__ positions, const uint16_t* __restrict__ cos_table,
    const uint16_t* __restrict__ sin_table, uint16_t* __restrict__ q_out, uint16_t* __restrict__ pair,
    int query_heads, int kv_heads, int D, int cap, int slot0, int zero_prefix) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const int heads = query_heads + 2 * kv_heads;
  const int W = heads * D;
  const int half = D >> 1;
  const int quads = half >> 2;
  const long long items = (long long)M * heads * quads;
  if (t < items) {
    const int dq = (int)(t % quads);
    const int h = (int)((t / quads) % heads);
    const int m = (int)(t / ((long long)quads * heads));
    const int d = 4 * dq;
    const size_t e = (size_t)m * W + (size_t)h * D + d;
    float a[4] = {0.f, 0.f, 0.f, 0.f}, b[4] = {0.f, 0.f, 0.f, 0.f};
    sum_partials(partials, splits, (size_t)M * W, e, a);
    sum_partials(partials, splits, (size_t)M * W, e + half, b);
    if (bias != nullptr) {
      const uint2 ba = *reinterpret_cast<const uint2*>(bias + (size_t)h * D + d);
      const uint2 bb = *reinterpret_cast<const uint2*>(bias + (size_t)h * D + d + half);
      a[0] += bf16_lo(ba.x);
      a[1] += bf16_hi(ba.x);
      a[2] += bf16_lo(ba.y);
      a[3] += bf16_hi(ba.y);
      b[0] += bf16_lo(bb.x);
      b[1] += bf16_hi(bb.x);
      b[2] += bf16_lo(bb.y);
      b[3] += bf16_hi(bb.y);
    }
    const uint2 ya = make_uint2(pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]));
    const uint2 yb = make_uint2(pack_bf16x2(b[0], b[1]), pack_bf16x2(b[2], b[3]));
    *reinterpret_cast<uint2*>(Y + e) = ya;
    *reinterpret_cast<uint2*>(Y + e + half) = yb;
    rope_quad_store(ya, yb, m, h, d, M, positions, cos_table, sin_table, q_out, pair, query_heads, kv_heads, D, cap,
                    slot0);
    return;
  }
  if (zero_prefix) rope_zero_prefix(t - items, pair, kv_heads, D, cap, slot0);
}

// RoPE and the cache fill from a stored projection y[m][W] (bias included): the
// values of aoto_rope_qkv_prefill (batch 1) with one thread per quad as in
// aoto_w4_gemm_reduce_rope, 8-byte loads and stores. Same outputs and limits
// (D % 8 == 0, y 8-byte aligned).
extern "C" __global__ __launch_bounds__(256) void aoto_rope_qkv_rows(
    const uint16_t* __restrict__ Y, int M, const long long* __restrict__ positions,
    const uint16_t* __restrict__ cos_table, const uint16_t* __restrict__ sin_table, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ pair, int query_heads, int kv_heads, int D, int cap, int slot0, int zero_prefix) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const int heads = query_heads + 2 * kv_heads;
  const int W = heads * D;
  const int half = D >> 1;
  const int quads = half >> 2;
  const long long items = (long long)M * heads * quads;
  if (t < items) {
    const int dq = (int)(t % quads);
    const int h = (int)((t / quads) % heads);
    const int m = (int)(t / ((long long)quads * heads));
    const int d = 4 * dq;
    const size_t e = (size_t)m * W + (size_t)h * D + d;
    const uint2 ya = *reinterpret_cast<const uint2*>(Y + e);
    const uint2 yb = *reinterpret_cast<const uint2*>(Y + e + half);
    rope_quad_store(ya, yb, m, h, d, M, positions, cos_table, sin_table, q_out, pair, query_heads, kv_heads, D, cap,
                    slot0);
    return;
  }
  if (zero_prefix) rope_zero_prefix(t - items, pair, kv_heads, D, cap, slot0);
}

// The paired form's split-K sum: gate = sum of partials[0 .. splits), up = sum
// of partials[splits .. 2 * splits), y = bf16(up * silu(bf16(gate))), one thread
// per 4 outputs (the gate's rounding and the up epilogue of the unpaired pair).
extern "C" __global__ __launch_bounds__(256) void aoto_w4_gemm_reduce_paired(const float* __restrict__ partials,
                                                                             int splits, uint16_t* __restrict__ Y,
                                                                             int M, int N) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long quads = (long long)M * N / 4;
  if (t >= quads) return;
  const size_t e = (size_t)t * 4;
  float g[4] = {0.f, 0.f, 0.f, 0.f}, v[4] = {0.f, 0.f, 0.f, 0.f};
  sum_partials(partials, splits, (size_t)M * N, e, g);
  sum_partials(partials + (size_t)splits * M * N, splits, (size_t)M * N, e, v);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float gr = round_bf16(g[i]);
    v[i] = v[i] * (gr / (1.0f + expf(-gr)));
  }
  uint2 o;
  o.x = pack_bf16x2(v[0], v[1]);
  o.y = pack_bf16x2(v[2], v[3]);
  *reinterpret_cast<uint2*>(Y + e) = o;
}

}  // namespace aoto

#define AOTO_GEMM_INSTANCE(BITS, TN, TM, BIAS, RES, GATE)                                                  \
  extern "C" __global__ __launch_bounds__(256) void                                                         \
      aoto_w##BITS##_gemm_n##TN##_m##TM##_b##BIAS##_r##RES##_g##GATE(                                       \
          const uint16_t* X, const aoto::GemmWord<BITS>::type* words, const uint16_t* scales,               \
          const uint16_t* bias, const uint16_t* residual, const uint16_t* gate, uint16_t* Y, int M, int N,  \
          int K, int group, int kslice, float* partials) {                                                  \
    aoto::w4_gemm_body<BITS, TN, TM, aoto::gemm_depth(TM), BIAS, RES, GATE>(X, words, scales, bias, residual, gate, Y, M, N, K,   \
                                                      group, kslice, partials);                             \
  }

#define AOTO_GEMM_EPILOGUES(BITS, TN, TM)      \
  AOTO_GEMM_INSTANCE(BITS, TN, TM, 0, 0, 0)    \
  AOTO_GEMM_INSTANCE(BITS, TN, TM, 1, 0, 0)    \
  AOTO_GEMM_INSTANCE(BITS, TN, TM, 0, 1, 0)    \
  AOTO_GEMM_INSTANCE(BITS, TN, TM, 0, 0, 1)
// aoto_w{BITS}_gemm_n{TN}_m{TM}_paired: the gate/up pair in one pass.
#define AOTO_GEMM_PAIRED_INSTANCE(BITS, TN, TM)                                                           \
  extern "C" __global__ __launch_bounds__(256) void aoto_w##BITS##_gemm_n##TN##_m##TM##_paired(            \
      const uint16_t* X, const aoto::GemmWord<BITS>::type* words, const uint16_t* scales,                  \
      const aoto::GemmWord<BITS>::type* up_words, const uint16_t* up_scales, uint16_t* Y, int M, int N,    \
      int K, int group, int kslice, float* partials) {                                                     \
    aoto::w4_gemm_body<BITS, TN, TM, aoto::gemm_depth(TM), false, false, false, true>(X, words, scales, nullptr, nullptr,       \
                                                                nullptr, Y, M, N, K, group, kslice,       \
                                                                partials, up_words, up_scales);           \
  }
// aoto_w{BITS}_gemm_n{TN}_m{TM}_rope_b{BIAS}: the unsplit q/k/v projection with
// its bias, RoPE and cache fill (block columns a whole number of heads).
#define AOTO_GEMM_ROPE_INSTANCE(BITS, TN, TM, BIAS)                                                         \
  extern "C" __global__ __launch_bounds__(256) void aoto_w##BITS##_gemm_n##TN##_m##TM##_rope_b##BIAS(        \
      const uint16_t* X, const aoto::GemmWord<BITS>::type* words, const uint16_t* scales,                    \
      const uint16_t* bias, uint16_t* Y, int M, int N, int K, int group, aoto::QkvRope rope) {               \
    aoto::w4_gemm_body<BITS, TN, TM, aoto::gemm_depth(TM), BIAS, false, false, false, true>(                 \
        X, words, scales, bias, nullptr, nullptr, Y, M, N, K, group, K, nullptr, nullptr, nullptr, rope);    \
  }
