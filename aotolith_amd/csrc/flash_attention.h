// Prefill GQA attention on bf16 MFMA (online softmax, one pass over K/V).
//
// Semantics (runtime/mlx_ops/attention.py:73-122, legalize/attention.py:105-170,
// mask from models/decoder.py:226-247):
//   O[b][i][h*D:(h+1)*D] = sum_j softmax_j(scale * q_i . k_j | keep(i, j)) v_j
// with key/value head h / (Hq/Hkv), f32 scores and softmax, P rounded to bf16
// before P.V (codegen/attention.py:367-371), and a query row whose keys are all
// masked giving 0 (safe_softmax).
// keep(i, j): with `mask` non-null, mask[b*mask_batch_stride + i*Mk + j] != 0;
// otherwise j >= key_start and, when `causal`, j <= i + (Mk - M) - the
// reference's prefill mask "causal and not a left pad" at key_start = M - length.
//
// Layout: q[B][Hq][M][D] (head-major, as the fused RoPE writes it); keys and
// values at k/v + b*kv_batch_stride + kvh*kv_head_stride + j*D; output
// [B][M][Hq*D] (the o projection's input rows).
//
// Block: 4 waves, 128 queries of one head (wave w: queries q0 + 32w .. q0 + 32w + 31);
// the short-prompt instances take 2 or 1 waves (64 or 32 queries) per key group.
// Key tiles of 64 rows are staged in LDS row-major, each with its own row stride
// so that its reads touch all 64 four-byte banks once per phase: K rows D + 8 bf16
// apart (a 16-byte read per lane, 16 lanes a phase: rows 4 banks apart), V rows
// D + 32 apart (the transpose reads' 4 rows of 16 banks start 16 banks apart).
// One stride D + 16 for both left every K and V read 2-way conflicted (rocprof
// SQ_LDS_BANK_CONFLICT = 128 cycles per wave and tile). Double-buffered: the next
// tile's global loads are in flight while the current tile is computed, one
// barrier per tile. Per wave and key tile, with v_mfma_f32_32x32x16_bf16:
//   S^T (2 x [32 keys x 32 queries]) = K . Q^T   A: K rows from LDS, B: Q in registers
//   O^T (D/32 x [32 d x 32 queries]) += V^T . P^T  A: V^T by LDS transpose reads
//                                                 (ds_read_b64_tr_b16), B: P from S^T
// Lane l owns query l % 32 in both products (C column), so the softmax state of a
// query lives in lanes l and l ^ 32, which hold the other half of its keys.
// The MFMA's k slots are a permutation of the tile's keys, the same for both
// operands: k-step t, slot (h = l / 32, j) holds key 16t + 8(j / 4) + 4h + j % 4,
// which is where S^T's C layout leaves that key in lane l.
// The softmax runs in base 2 with log2(e) folded into the scale. Two blocks share a
// CU (256 VGPRs a lane at most, two 4-wave blocks of LDS), so one block's softmax
// overlaps the other's products.
#pragma once

#include <type_traits>

#include "common.h"

namespace aoto {

typedef __bf16 fa_bf16x8 __attribute__((ext_vector_type(8)));
typedef float fa_f32x16 __attribute__((ext_vector_type(16)));
typedef short fa_s16x4 __attribute__((ext_vector_type(4)));
typedef short fa_s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) fa_s16x4 fa_lds_s16x4;

constexpr int kFlashQueries = 128;  // queries per block
constexpr int kFlashKeys = 64;      // keys per staged tile

// Two LDS transpose reads give lane l the A operand of O^T's k-step `t` for the
// 32 d rows starting at `d_base`: V[key][d] for d = d_base + l % 32 and the keys of
// slots (l / 32, j). In each 16-lane group lane r addresses the 8 bytes at
// V[kb + r / 4][d0 + 4 (r % 4)]; the transpose hands lane i element i % 4 of the
// chunks of lanes i / 4 + 4m (m = 0..3), i.e. V[kb + m][d0 + i].
template <int STR>
AOTO_DEVICE fa_bf16x8 flash_v_operand(const uint16_t* vs, int t, int d_base, int lane) {
  const int group = lane >> 4, r = lane & 15, half = lane >> 5;
  const int d0 = d_base + 16 * (group & 1) + 4 * (r & 3);
  const int row = 16 * t + 4 * half + (r >> 2);
  const uint16_t* p0 = vs + row * STR + d0;
  const fa_s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fa_lds_s16x4*)(p0));
  const fa_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fa_lds_s16x4*)(p0 + 8 * STR));
  // concatenated as vectors: through a short[8] the compiler merges halves with a
  // v_bfi per read, and each merge waits for its read (the reads then retire one by one)
  const fa_s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(fa_bf16x8, both);
}

// MASKED: the explicit-mask form (a separate instance, so the causal form carries
// no mask registers).
// KG key groups: with KG = 2 the block has 8 waves, two groups of 4 over the same
// 128 queries; group g takes the g-th half of the block's key tiles, with its own
// double-buffered K/V stages, and after the loop group 1 hands its softmax state
// (reference max, sum, O) to group 0 through LDS, which combines the two as the
// split merge of decode attention does. A CU then always holds two waves per SIMD
// - one block of 8, where two 4-wave blocks would leave the heavy causal tile alone
// once its light partner ends - and a q-tile's keys take half the time.
// QW waves per key group, 32 queries each (BQ = 32 QW queries per block): 4 in the
// ordinary instances; 2 in the short-prompt instance, which spreads a short prompt's
// few blocks over twice the CUs (one wave per SIMD instead of two sharing its MFMA pipe).
template <int D, int KG, bool MASKED, int QW = 4>
__device__ void flash_attention_body(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                     const uint16_t* __restrict__ v, long long kv_batch_stride,
                                     long long kv_head_stride, const uint8_t* __restrict__ mask,
                                     long long mask_batch_stride, int causal, int key_start, int M, int Mk,
                                     int batch, int query_heads, int kv_heads, float scale,
                                     uint16_t* __restrict__ out) {
  constexpr int BQ = 32 * QW, BK = kFlashKeys;
  constexpr int GT = 64 * QW;              // threads per key group
  static_assert(QW != 4 || BQ == kFlashQueries, "the ordinary instances take kFlashQueries queries");
  constexpr int STRK = D + 8;              // bf16 per staged K row
  constexpr int STRV = D + 32;             // bf16 per staged V row
  constexpr int VOFF = BK * STRK;          // V tile after the K tile in a stage
  constexpr int DS = D / 16;               // k-steps of S^T (16 d each)
  constexpr int DT = D / 32;               // 32-row d tiles of O^T
  constexpr int CHUNKS = BK * D / 8;       // 16-byte chunks of one K (or V) tile
  constexpr int PER = 2 * CHUNKS / GT;     // chunks per thread per tile, K then V
  static_assert(PER == DS || PER % (2 * DS) == 0, "tile loads spread evenly over the S^T products");
  constexpr int ROW_CHUNKS = D / 8;
  __shared__ __attribute__((aligned(16))) uint16_t lds_all[KG][2][BK * (STRK + STRV)];
  // wave and group are uniform per wave; saying so (readfirstlane) keeps the tile
  // loop's branches scalar - as exec-masked branches their paths merged, and the
  // loads of one path made the other wait for them
  const int group = KG == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)threadIdx.x / GT);
  const int lt = (int)threadIdx.x % GT;  // thread index within the group
  auto& lds = lds_all[group];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6) % QW);
  const int col = lane & 31, half = lane >> 5;
  // Query tiles in the order T-1, T-2, ..., T/2 (heaviest first), then 0, 1, ...:
  // blocks are dealt to the 8 XCDs round robin and to each XCD's CUs in turn, so the
  // block that takes a CU's second slot comes from the second half of the order and
  // each CU gets a heavy and a light tile of the causal triangle. With a multiple of
  // 8 query heads the heads of one kv group go to one XCD, so their K/V stays in
  // that XCD's L2.
  const int bh_count = batch * query_heads;
  const int tiles_q = (M + BQ - 1) / BQ;
  const int rank = (int)blockIdx.x / bh_count;
  // (KG = 2: one block per CU, so the second round of blocks goes to the CUs that
  // finish first - heaviest first throughout pairs each heavy tile with a light one.)
  const int qt = KG == 2 ? tiles_q - 1 - rank : (rank < tiles_q / 2 ? tiles_q - 1 - rank : rank - tiles_q / 2);
  const int slot = (int)blockIdx.x % bh_count;
  const int b = slot / query_heads;
  const int hs = slot % query_heads;
  const int h = (query_heads % 8 == 0) ? (hs % 8) * (query_heads / 8) + hs / 8 : hs;
  const int kvh = h / (query_heads / kv_heads);
  const int q0 = qt * BQ;
  const int qa = q0 + wave * 32;           // this wave's first query
  const int qi = qa + col;                 // this lane's query
  const int qrow = min(qi, M - 1);
  const int shift = Mk - M;

  const uint16_t* kh = k + (size_t)b * kv_batch_stride + (size_t)kvh * kv_head_stride;
  const uint16_t* vh = v + (size_t)b * kv_batch_stride + (size_t)kvh * kv_head_stride;

  // Q^T operand: query qi, d = 16 s + 8 half + j.
  fa_bf16x8 qf[DS];
  {
    const uint16_t* qp = q + (((size_t)b * query_heads + h) * M + qrow) * D + 8 * half;
#pragma unroll
    for (int s = 0; s < DS; ++s) qf[s] = *reinterpret_cast<const fa_bf16x8*>(qp + 16 * s);
  }

  // Keys this block can see.
  const int j_lo = MASKED ? 0 : max(0, key_start);
  int j_hi = Mk;
  if (!MASKED && causal) j_hi = min(Mk, q0 + BQ + shift);
  const int tile_begin0 = (j_lo / BK) * BK;
  const int n_all = j_hi > tile_begin0 ? (j_hi - tile_begin0 + BK - 1) / BK : 0;
  // this group's contiguous share of the key tiles; both groups run the longer
  // share's trip count (every thread meets every barrier)
  const int share = (n_all + KG - 1) / KG;
  const int tile_begin = tile_begin0 + group * share * BK;
  const int n_tiles = max(0, min(share, n_all - group * share));
  const int trips = share;

  // Rows outside [key_start, Mk) (without an explicit mask) are staged as zeros, so
  // a masked key's value never meets P (0 * NaN would poison the row); tiles wholly
  // inside are stored without that test. The load address is clamped into the
  // head (no branch or wait around the loads themselves).
  auto load_one = [&](int i, int j0, uint4 (&reg)[PER]) {
    const int c = lt + (i % (PER / 2)) * GT;
    const int row = c / ROW_CHUNKS, cc = c % ROW_CHUNKS;
    const uint16_t* base = i < PER / 2 ? kh : vh;
    reg[i] = *reinterpret_cast<const uint4*>(base + (size_t)min(j0 + row, Mk - 1) * D + cc * 8);
  };
  auto load_tile = [&](int j0, uint4 (&reg)[PER]) {
#pragma unroll
    for (int i = 0; i < PER; ++i) load_one(i, j0, reg);
  };
  auto store_tile = [&](int buffer, int j0, const uint4 (&reg)[PER]) {
    auto slot = [&](int i) {
      const int c = lt + (i % (PER / 2)) * GT;
      const int row = c / ROW_CHUNKS, cc = c % ROW_CHUNKS;
      return reinterpret_cast<uint4*>(&lds[buffer][i < PER / 2 ? row * STRK : VOFF + row * STRV] + cc * 8);
    };
    if (j0 + BK <= Mk && (MASKED || j0 >= key_start)) {
#pragma unroll
      for (int i = 0; i < PER; ++i) *slot(i) = reg[i];
    } else {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int j = j0 + (lt + (i % (PER / 2)) * GT) / ROW_CHUNKS;
        // zeroed by a mask, not a select: a select became a branch around register copies
        const uint32_t keep = (j < Mk && (MASKED || j >= key_start)) ? 0xFFFFFFFFu : 0u;
        *slot(i) = make_uint4(reg[i].x & keep, reg[i].y & keep, reg[i].z & keep, reg[i].w & keep);
      }
    }
  };

  const float c2 = scale * 1.4426950408889634f;  // scores in log2 units
  fa_f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = fa_f32x16{};
  float run_max = -INFINITY, run_sum = 0.f;

  // Tile t from stage `cur`, and the loads of the tile at `jn` into `stage`: one
  // load after every second S^T product (2·DS products, PER = DS loads), so the
  // CU's address path works through the next tile's 32 KB per group while the
  // products run - issued all at once after the barrier, the eight waves' loads
  // queued there for ~0.5 us (a fifth of the interval) before the first product.
  // Every wave computes every trip: a tile past the group's share (t >= n_tiles,
  // the stage then holds a clamped copy) or past the wave's causal edge is fully
  // masked (p = 0). Skipping it put the next tile's loads on two paths, and the
  // compiler's wait counting, merging them, made the computing path wait for them.
  // `prefetch` (a compile-time bool) is false for the last trip, which loads nothing.
  auto compute_tile = [&](int t, int cur, int jn, uint4 (&stage)[PER], auto prefetch) {
    const int j0 = tile_begin + t * BK;
    const bool real = t < n_tiles;
    {
      const uint16_t* ks = lds[cur];
      const uint16_t* vs = lds[cur] + VOFF;
      fa_f32x16 sacc[2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        sacc[sub] = fa_f32x16{};
#pragma unroll
        for (int s = 0; s < DS; ++s) {
          const fa_bf16x8 a = *reinterpret_cast<const fa_bf16x8*>(ks + (sub * 32 + col) * STRK + 16 * s + 8 * half);
          sacc[sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[s], sacc[sub], 0, 0, 0);
          if constexpr (decltype(prefetch)::value) {
            if constexpr (PER >= 2 * DS) {
#pragma unroll
              for (int u = 0; u < PER / (2 * DS); ++u) load_one((sub * DS + s) * (PER / (2 * DS)) + u, jn, stage);
            } else if ((sub * DS + s) & 1) {
              load_one((sub * DS + s) >> 1, jn, stage);
            }
          }
        }
      }
      // Scores of key j0 + 32 sub + 8 (e / 4) + 4 half + e % 4 for query qi; only
      // tiles that straddle the causal diagonal, the left pad or the end of the keys
      // (or any tile, with an explicit mask) test each key.
      const bool whole = !MASKED && real && j0 >= key_start && j0 + BK <= Mk && (!causal || j0 + BK - 1 <= qa + shift);
      if (!whole) {
        const int key0 = j0 + 4 * half;
        if constexpr (MASKED) {
          const uint8_t* mrow = mask + (size_t)b * mask_batch_stride + (size_t)qrow * Mk;
#pragma unroll
          for (int sub = 0; sub < 2; ++sub) {
            uint32_t keep[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int j = key0 + 32 * sub + 8 * (e >> 2) + (e & 3);
              keep[e] = (real && j < Mk) ? mrow[min(j, Mk - 1)] : 0u;
            }
#pragma unroll
            for (int e = 0; e < 16; ++e)
              if (!keep[e]) sacc[sub][e] = -INFINITY;
          }
        } else {
          // key key0 + c is kept for lo <= c <= hi; c is a constant per element, so
          // the tests compare against two registers instead of 32 key indices
          const int lo = key_start - key0;
          const int hi = real ? (causal ? min(Mk - 1, qi + shift) : Mk - 1) - key0 : -1;
#pragma unroll
          for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int c = 32 * sub + 8 * (e >> 2) + (e & 3);
              if (c < lo || c > hi) sacc[sub][e] = -INFINITY;
            }
        }
      }
      // Raw scores; the scale (> 0) is applied to the maximum and inside the exponent's FMA.
      float tile_max = -INFINITY;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e) tile_max = fmaxf(tile_max, sacc[sub][e]);
      tile_max *= c2;
      // The exponentials' reference point moves only when a score passes it by more
      // than 8 (in log2 units), so p stays below 2^8 and O (D/2 accumulators a lane)
      // is rescaled on few tiles; the final division by the sum is unchanged.
      tile_max = xor32_max(tile_max);
      const float moved = tile_max > run_max + 8.f ? tile_max : run_max;
      const float correction = moved == run_max ? 1.f : __builtin_amdgcn_exp2f(run_max - moved);
      run_max = moved;
      const float ref = moved == -INFINITY ? 0.f : moved;
      if (__any(correction != 1.f)) {
        run_sum *= correction;
#pragma unroll
        for (int d = 0; d < DT; ++d) o[d] *= correction;
      }
      // P (bf16) as the B operand of k-step kt: elements 8 (kt % 2) .. +7 of sacc[kt / 2].
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        float p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt >> 1][8 * (kt & 1) + j], c2, -ref));
          run_sum += p[j];
        }
        const uint32_t packed[4] = {cvt_pk_bf16(p[0], p[1]), cvt_pk_bf16(p[2], p[3]), cvt_pk_bf16(p[4], p[5]),
                                    cvt_pk_bf16(p[6], p[7])};
        const fa_bf16x8 pb = __builtin_bit_cast(fa_bf16x8, packed);
#pragma unroll
        for (int d = 0; d < DT; ++d)
          o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(flash_v_operand<STRV>(vs, kt, 32 * d, lane), pb, o[d], 0,
                                                          0, 0);
      }
    }
  };

  // The first stage is written even for a group without tiles: every trip computes
  // (fully masked past the share), and P = 0 meeting uninitialized LDS in V could
  // meet a NaN bit pattern; clamped rows hold keys, rows outside them zeros.
  uint4 stage[PER];
  load_tile(tile_begin, stage);
  store_tile(0, tile_begin, stage);
  // Nothing may be pending when the loop starts: a Q load the compiler's wait
  // counting believed still in flight would make every S^T product below wait for
  // the next tile's prefetch (loads retire in issue order).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // The next tile's loads and stores are unconditional - past the group's share a
  // clamped tile goes into the stage no product reads again (its last reads ended
  // before the previous barrier) - so the compiler's wait counting sees the same
  // loads on every path: with a conditional store it assumed loads still in
  // flight at the loop head and waited for them before reusing their registers.
  // The last trip is peeled: it issues no loads and stores no stage, so it does not
  // wait for a memory round trip before its barrier (a one-trip block - a short
  // prompt - otherwise fetched its tile twice).
  const int last_tile = max(n_tiles - 1, 0);
  for (int t = 0; t + 1 < trips; ++t) {
    const int jn = tile_begin + min(t + 1, last_tile) * BK;
    compute_tile(t, t & 1, jn, stage, std::true_type{});
    store_tile((t + 1) & 1, jn, stage);
    __syncthreads();
  }
  if (trips > 0) {
    compute_tile(trips - 1, (trips - 1) & 1, 0, stage, std::false_type{});
    __syncthreads();
  }

  if constexpr (KG == 2) {
    // group 1's state into its own stages (dead: the loop ended on a barrier), then
    // group 0 combines it with its own, lane by lane (same query, same d)
    constexpr int REC = 2 + 16 * DT;
    static_assert(QW * 64 * REC * 4 <= (int)sizeof(lds_all[1]), "the handover fits group 1's stages");
    float* hand = reinterpret_cast<float*>(&lds_all[1][0][0]) + (size_t)(wave * 64 + lane) * REC;
    if (group == 1) {
      hand[0] = run_max;
      hand[1] = run_sum;
#pragma unroll
      for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int e = 0; e < 16; ++e) hand[2 + 16 * d + e] = o[d][e];
    }
    __syncthreads();
    if (group == 1) return;
    const float m1 = hand[0], s1 = hand[1];
    const float big = fmaxf(run_max, m1);
    const float a0 = (big == -INFINITY || run_max == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(run_max - big);
    const float a1 = (big == -INFINITY || m1 == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m1 - big);
    run_sum = run_sum * a0 + s1 * a1;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[d][e] = o[d][e] * a0 + hand[2 + 16 * d + e] * a1;
  }
  const float total = xor32_sum(run_sum);
  if (qi >= M) return;
  const float inv = total > 0.f ? 1.0f / total : 0.f;
  uint16_t* orow = out + ((size_t)b * M + qi) * ((size_t)query_heads * D) + (size_t)h * D + 4 * half;
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint2 w;
      w.x = pack_bf16x2(o[d][4 * g] * inv, o[d][4 * g + 1] * inv);
      w.y = pack_bf16x2(o[d][4 * g + 2] * inv, o[d][4 * g + 3] * inv);
      *reinterpret_cast<uint2*>(orow + 32 * d + 8 * g) = w;
    }
}

}  // namespace aoto

// aoto_flash_attention_d{D} (4-wave blocks, two per CU) and aoto_flash_attention_d{D}_k2
// (8-wave blocks whose two wave groups split the keys); the _m forms take an explicit mask.
#define AOTO_FLASH_INSTANCE_KG(D, KG, MASKED, SUFFIX, MINB, QW)                                         \
  extern "C" __global__ __launch_bounds__(64 * QW * KG, MINB) void aoto_flash_attention_d##D##SUFFIX(   \
      const uint16_t* q, const uint16_t* k, const uint16_t* v, long long kv_batch_stride,               \
      long long kv_head_stride, const uint8_t* mask, long long mask_batch_stride, int causal,           \
      int key_start, int M, int Mk, int batch, int query_heads, int kv_heads, float scale,              \
      uint16_t* out) {                                                                                  \
    aoto::flash_attention_body<D, KG, MASKED, QW>(q, k, v, kv_batch_stride, kv_head_stride, mask, mask_batch_stride, \
                                      causal, key_start, M, Mk, batch, query_heads, kv_heads, scale, out); \
  }
#define AOTO_FLASH_INSTANCE(D)                   \
  AOTO_FLASH_INSTANCE_KG(D, 1, false, , 2, 4)    \
  AOTO_FLASH_INSTANCE_KG(D, 2, false, _k2, 1, 4) \
  AOTO_FLASH_INSTANCE_KG(D, 1, true, _m, 2, 4)   \
  AOTO_FLASH_INSTANCE_KG(D, 2, true, _k2_m, 1, 4)
