// Wave-persistent, software-pipelined form of the W4 decode GEMV (same semantics
// and rounding points as w4_gemv.h).
//
// Why a second form: at decode shapes the plain kernel is latency-bound. Each
// block stages x (and the RMSNorm statistics) behind block barriers before it
// issues a weight load, and its loop waits for every outstanding load before
// the first dot product. Here
//   * a lane's whole share of a row (CPL 16-byte chunks: chunk li + LPR*j of the
//     row, and their group scales) is loaded with unconditional, clamped loads,
//     so the compiler counts them statically;
//   * the first tile's loads are issued before x is staged, so the staging
//     latency hides under them;
//   * each wave stages x (and the norm) into its own LDS region with wave-level
//     reductions only - no block barrier anywhere, so small grids use 1-wave
//     blocks spread over more CUs;
//   * waves are persistent: tile t+waves is loaded while tile t is reduced, so a
//     wave keeps 2*CPL chunks in flight and stages x once for many rows;
//   * nibbles become bf16 (136 + code) pairs with one v_bitop3 each (mask,
//     bias-by-8 and the 0x4300 exponent in one three-input op), 11 VALU ops per
//     packed word including the four v_dot2_f32_bf16.
#pragma once

#include "common.h"
#include "w4_gemv.h"
#include "gemv_finish_args.h"

namespace aoto {

// (136 + code) bf16 pairs of one nibble position pair, straight from the raw
// word: bitop3 with table 0x6A computes (t & m) ^ (c & m) | (c & ~m) per bit for
// m = 0x000F000F, c = 0x43084308 - the nibble, its top bit flipped (code + 8),
// under the 0x4300 exponent.
AOTO_DEVICE uint32_t nibble_pair(uint32_t t) {
  return __builtin_amdgcn_bitop3_b32(t, 0x000F000Fu, 0x43084308u, 0x6A);
}

AOTO_DEVICE float chunk_dot_fast(const uint4 q, const uint4* __restrict__ xc) {
  const uint32_t words[4] = {q.x, q.y, q.z, q.w};
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t t = words[j];
    const uint4 xv = xc[j];
    acc = dot2_bf16(nibble_pair(t), xv.x, acc);
    acc = dot2_bf16(nibble_pair(t >> 4), xv.y, acc);
    acc = dot2_bf16(nibble_pair(t >> 8), xv.z, acc);
    acc = dot2_bf16(nibble_pair(t >> 12), xv.w, acc);
  }
  return acc;
}

// One 16-byte vector of x, bf16 pairs (e0,e1) .. (e6,e7): with NORM scaled by
// the RMS factor ns and multiplied by the norm weight's vector, each product
// rounded once to bf16; repacked in dot2 pair order {(e0,e4), (e1,e5), (e2,e6),
// (e3,e7)}. Returns `corr` plus 136 times the (rounded) values - the offset the
// (136 + code) weight pairs add to a dot product - accumulated with dot2
// against the bf16 pair (136, 136) (each product 136 * x is exact).
constexpr uint32_t kBf16Pair136 = 0x43084308u;
template <bool NORM>
AOTO_DEVICE float pack_x8(const uint4 raw, const uint4 w, float ns, uint4& out, float corr = 0.f) {
  const uint32_t r[4] = {raw.x, raw.y, raw.z, raw.w};
  if (NORM) {
    const uint32_t wr[4] = {w.x, w.y, w.z, w.w};
    float lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      lo[k] = (ns * bf16_lo(r[k])) * bf16_lo(wr[k]);
      hi[k] = (ns * bf16_hi(r[k])) * bf16_hi(wr[k]);
    }
    // element 2k is lo[k], 2k+1 is hi[k]
    out = make_uint4(cvt_pk_bf16(lo[0], lo[2]), cvt_pk_bf16(hi[0], hi[2]), cvt_pk_bf16(lo[1], lo[3]),
                     cvt_pk_bf16(hi[1], hi[3]));
  } else {
    out = make_uint4(__builtin_amdgcn_perm(r[2], r[0], 0x05040100u), __builtin_amdgcn_perm(r[2], r[0], 0x07060302u),
                     __builtin_amdgcn_perm(r[3], r[1], 0x05040100u), __builtin_amdgcn_perm(r[3], r[1], 0x07060302u));
  }
  corr = dot2_bf16(out.x, kBf16Pair136, corr);
  corr = dot2_bf16(out.y, kBf16Pair136, corr);
  corr = dot2_bf16(out.z, kBf16Pair136, corr);
  return dot2_bf16(out.w, kBf16Pair136, corr);
}

// Sum of squares of the eight bf16 values of a 16-byte vector (each square is
// exact in f32), accumulated with dot2.
AOTO_DEVICE float sum_squares8(const uint4 raw, float ss) {
  ss = dot2_bf16(raw.x, raw.x, ss);
  ss = dot2_bf16(raw.y, raw.y, ss);
  ss = dot2_bf16(raw.z, raw.z, ss);
  return dot2_bf16(raw.w, raw.w, ss);
}

// x (optionally RMS-normalized and rounded to bf16) staged into LDS, in dot2 pair
// order, plus per-chunk offsets (136 x the chunk's sum, pack_x8). Split in two like
// DirectActivation: issue() loads all of x (and the norm weight) - XV 16-byte
// vectors per thread - and finish() packs and stores it. The caller issues x
// first and the first tile's weights right after, so the wait for x is a wait for
// x alone (loads return in issue order) while the weights are already in flight.
// WAVE: each wave stages its own copy with wave-level reductions only (no block
// barrier; XV >= K/512). Otherwise one copy per block of kGemvThreads threads,
// whose RMS statistic is a block sum (a barrier; XV >= K/2048): for long
// reductions (K = 4096, 14336) a per-wave copy would cost as many LDS writes and
// cache reads as the wave's share of the weights.
template <bool NORM, int XV, bool WAVE>
struct StagedActivation {
  uint4 xr[XV];
  uint4 wr[NORM ? XV : 1];

  AOTO_DEVICE static int index(int i) { return WAVE ? (int)(threadIdx.x & 63) + 64 * i
                                                     : (int)threadIdx.x + kGemvThreads * i; }

  AOTO_DEVICE void issue(const uint16_t* __restrict__ x, const uint16_t* __restrict__ norm_w, int K) {
    issue_x(x, K);
    issue_norm(norm_w, K);
  }
  // zero: stage a zero vector instead of x (x is still a valid address)
  AOTO_DEVICE void issue_x(const uint16_t* __restrict__ x, int K, bool zero = false) {
    const int vecs = K >> 3;
    const uint4* xv = reinterpret_cast<const uint4*>(x);
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const uint4 v = xv[min(index(i), vecs - 1)];
      xr[i] = zero ? make_uint4(0u, 0u, 0u, 0u) : v;
    }
  }
  AOTO_DEVICE void issue_norm(const uint16_t* __restrict__ norm_w, int K) {
    const int vecs = K >> 3;
    const uint4* wv = reinterpret_cast<const uint4*>(norm_w);
    if (NORM) {
#pragma unroll
      for (int i = 0; i < XV; ++i) wr[i] = wv[min(index(i), vecs - 1)];
    }
  }

  AOTO_DEVICE void finish(float eps, int K, uint4* __restrict__ xp, float* __restrict__ csum) const {
    const int vecs = K >> 3;
    float ns = 1.f;
    if (NORM) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < XV; ++i)
        if (index(i) < vecs) ss = sum_squares8(xr[i], ss);
      if (WAVE) {
        ss = wave_sum(ss);
      } else {
        __shared__ float scratch[kGemvThreads / 64];
        ss = block_sum<kGemvThreads>(ss, scratch);
      }
      ns = 1.0f / sqrtf(ss / (float)K + eps);
    }
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int v = index(i);
      uint4 packed;
      float sum = pack_x8<NORM>(xr[i], wr[NORM ? i : 0], ns, packed);
      if (v < vecs) xp[v] = packed;
      // A chunk (32 codes) is four consecutive vectors: threads 4c .. 4c+3.
      sum = group_sum<4>(sum);
      if (v < vecs && (v & 3) == 0) csum[v >> 2] = sum;
    }
    if (WAVE) {
      // no block barrier: the wave's LDS accesses are ordered among themselves
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else {
      __syncthreads();
    }
  }
};

// Direct staging for the latency-bound shapes: the LPR lanes of a row group hold,
// between them, every chunk of x (chunk li + LPR*j), so each lane loads just its
// own chunks (and the norm weight's) from global memory, the RMS statistic is a
// group sum over the LPR lanes, and the normalized pairs go straight into
// registers - no LDS and no wave-wide staging loop. Split in two so the x loads
// can be issued before the weight loads: loads return in issue order, so the
// norm statistic then waits for x alone, not for the weights behind it.
template <int LPR, int CPL, bool NORM>
struct DirectActivation {
  uint4 raw[CPL][4];
  uint4 wraw[NORM ? CPL : 1][4];

  AOTO_DEVICE void issue(const uint16_t* __restrict__ x, const uint16_t* __restrict__ norm_w, int K, int li) {
    const int nchunks = K >> 5;
    const uint4* xv = reinterpret_cast<const uint4*>(x);
    const uint4* wv = reinterpret_cast<const uint4*>(norm_w);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = min(li + LPR * j, nchunks - 1);
#pragma unroll
      for (int k = 0; k < 4; ++k) raw[j][k] = xv[c * 4 + k];
      if (NORM) {
#pragma unroll
        for (int k = 0; k < 4; ++k) wraw[j][k] = wv[c * 4 + k];
      }
    }
  }

  AOTO_DEVICE void finish(float eps, int K, int li, uint4 (&xr)[CPL][4], float (&cr)[CPL]) const {
    const int nchunks = K >> 5;
    float ns = 1.f;
    if (NORM) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if (li + LPR * j < nchunks) {
#pragma unroll
          for (int k = 0; k < 4; ++k) ss = sum_squares8(raw[j][k], ss);
        }
      }
      ss = group_sum<LPR>(ss);
      ns = 1.0f / sqrtf(ss / (float)K + eps);
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) sum = pack_x8<NORM>(raw[j][k], wraw[NORM ? j : 0][k], ns, xr[j][k], sum);
      cr[j] = sum;
    }
  }
};

// Wave-persistent body: wave w of the grid handles row tiles w, w + waves, ...;
// a tile is 64/LPR rows, LPR lanes per row, CPL chunks (16 B) per lane.
// waves_per_block is the launch's block size / 64, passed in because reading
// blockDim costs a memory round trip at kernel start.
// XREG: after staging, each lane copies the x chunks it uses (the same CPL
// chunks for every row it visits) into registers, so the row loop reads no LDS.
// XV == 0 selects direct staging (DirectActivation; x always in registers).
// ARGMAX: also reduce the wave's rows to one greedy-argmax key (argmax_key of
// the stored bf16 value and its row) and store it at keys[global wave index],
// 0 for a wave without rows; aoto_argmax_finish reduces the keys.
// BLOCKX: x staged once per block (StagedActivation; XV >= K/2048) into
// one LDS region the block's waves share; needs 4-wave blocks. With XREG the
// lanes copy their chunks out of it after the block's staging barrier.
// FINISH (block-staged forms): x is the embedding table and `keys` the previous
// LM head's argmax keys (GemvFinishArgs above).
template <int LPR, int CPL, int XV, bool XREG, bool NORM, bool PAIRED, bool BIAS, bool ARGMAX, bool BLOCKX = false,
          bool FINISH = false>
__device__ void w4_gemv_stream_body(const uint16_t* __restrict__ x, const uint4* __restrict__ words,
                                    const uint16_t* __restrict__ scales, const uint4* __restrict__ up_words,
                                    const uint16_t* __restrict__ up_scales, const uint16_t* __restrict__ norm_w,
                                    float eps, const uint16_t* __restrict__ bias, float alpha, float beta,
                                    uint16_t* __restrict__ y, int K, int N, int group_shift,
                                    int waves_per_block, unsigned long long* __restrict__ keys,
                                    const GemvFinishArgs& fin = GemvFinishArgs{}) {
  static_assert(!FINISH || (BLOCKX && !ARGMAX), "the finish prologue is a block-staged GEMV's");
  extern __shared__ uint4 lds[];
  constexpr int RPW = 64 / LPR;  // rows per wave tile
  const int nchunks = K >> 5;
  const int ngroups = nchunks >> group_shift;
  // readfirstlane: the wave index is uniform, and saying so keeps the tile loop
  // on scalar branches instead of exec-masked ones.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & (LPR - 1);
  const int rsub = lane / LPR;
  const int tiles = (N + RPW - 1) / RPW;
  const int total_waves = gridDim.x * waves_per_block;
  // Per-wave LDS region: K/8 pair vectors then K/32 chunk sums.
  const int region = (K >> 3) + ((K >> 5) + 3) / 4;
  uint4* xp = lds + (BLOCKX ? 0 : wave * region);
  float* csum = reinterpret_cast<float*>(xp + (K >> 3));

  int cidx[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) cidx[j] = min(li + LPR * j, nchunks - 1);

  // Two register sets, A and B, ping-pong across tiles: the loads for the next
  // tile go into one set while the other is consumed, so no loaded register is
  // ever copied (a copy would force a wait on every outstanding load) and scales
  // stay raw bits until use (a conversion right after the load would wait for
  // it). Loads are unconditional (row index clamped); the epilogue's bias /
  // residual element is loaded with the row's weights, not after the reduction.
  // A wave's last tile issues no prefetch.
  // Scales and bias are read as the aligned 32-bit pair holding the wanted bf16
  // (the host guarantees K/group and, with a bias, N are even, so the pair is in
  // bounds): a 16-bit load would be zero-extended where the register sets
  // change roles, which waits for the prefetch. With K/group even, a lane's
  // scale half is the same for every row.
  struct Regs {
    uint4 q[CPL];
    uint4 u[PAIRED ? CPL : 1];
    uint32_t s[CPL];
    uint32_t us[PAIRED ? CPL : 1];
    uint32_t b;
  };
  const uint32_t* scale_words = reinterpret_cast<const uint32_t*>(scales);
  const uint32_t* up_scale_words = reinterpret_cast<const uint32_t*>(up_scales);
  const uint32_t* bias_words = reinterpret_cast<const uint32_t*>(bias);
  // bf16 in the low half of a pair becomes f32 by << 16, in the high half by masking.
  auto pair_half = [](uint32_t pair, int high) {
    return __uint_as_float(high ? (pair & 0xFFFF0000u) : (pair << 16));
  };
  int shalf[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) shalf[j] = (cidx[j] >> group_shift) & 1;
  Regs ra, rb;

  auto load = [&](int tile, Regs& r) {
    const int row = min(min(tile, tiles - 1) * RPW + rsub, N - 1);
    const uint4* wrow = words + (size_t)row * nchunks;
    const uint32_t* srow = scale_words + (size_t)row * (ngroups >> 1);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if (ARGMAX) {
        // The greedy loop's LM head streams 68 MB per token once: non-temporal
        // loads keep it from evicting the layer weights the next token reads
        // again (+0.7% decode tok/s on the Qwen2-0.5B loop, same head time).
        typedef unsigned v4u __attribute__((ext_vector_type(4)));
        const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(wrow + cidx[j]));
        r.q[j] = make_uint4(t.x, t.y, t.z, t.w);
      } else {
        r.q[j] = wrow[cidx[j]];
      }
    }
    if (PAIRED) {
      const uint4* urow = up_words + (size_t)row * nchunks;
#pragma unroll
      for (int j = 0; j < CPL; ++j) r.u[j] = urow[cidx[j]];
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) r.s[j] = srow[cidx[j] >> (group_shift + 1)];
    if (PAIRED) {
      const uint32_t* usrow = up_scale_words + (size_t)row * (ngroups >> 1);
#pragma unroll
      for (int j = 0; j < CPL; ++j) r.us[j] = usrow[cidx[j] >> (group_shift + 1)];
    }
    if (BIAS) r.b = bias_words[row >> 1];
  };

  constexpr bool DIRECT = XV == 0;
  constexpr bool INREG = XREG || DIRECT;
  uint4 xr[INREG ? CPL : 1][4];
  float cr[INREG ? CPL : 1];

  unsigned long long best = 0;
  auto consume = [&](int tile, const Regs& r) {
    float total = 0.f, total_up = 0.f;
    // Branch-free over the chunks: a lane past the row's last chunk computes on
    // the clamped (in-bounds) chunk and weights it by zero. An exec-masked
    // branch here would hide the per-set load waits from the compiler's wait
    // placement, which then waits for the next tile's prefetch at the loop head.
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const bool valid = li + LPR * j < nchunks;
      const int c = cidx[j];
      const uint4* xc = INREG ? xr[j] : xp + c * 4;
      const float corr = INREG ? cr[j] : csum[c];
      total = fmaf(chunk_dot_fast(r.q[j], xc) - corr, valid ? pair_half(r.s[j], shalf[j]) : 0.f, total);
      if (PAIRED)
        total_up = fmaf(chunk_dot_fast(r.u[j], xc) - corr, valid ? pair_half(r.us[j], shalf[j]) : 0.f, total_up);
    }
    total = group_sum<LPR>(total);
    if (PAIRED) total_up = group_sum<LPR>(total_up);
    const int row = tile * RPW + rsub;
    if (li == 0 && row < N) {
      float out;
      if (PAIRED) {
        const float g = round_bf16(total);
        out = total_up * (g / (1.0f + expf(-g)));
      } else if (BIAS) {
        out = beta * pair_half(r.b, row & 1) + alpha * total;
      } else {
        out = total;
      }
      const uint32_t bits = f32_to_bf16(out);
      y[row] = (uint16_t)bits;
      if (ARGMAX) best = max_u64(best, argmax_key(bits, row));
    }
  };

  int tile = blockIdx.x * waves_per_block + wave;
  if constexpr (BLOCKX && FINISH) {
    // The first tile's loads, the norm weight and the keys (and block 0's step
    // state, history length and, once the position is known, RoPE rows), then
    // the token's embedding row as x.
    StagedActivation<NORM, (XV > 0 ? XV : 1), false> act;
    load(tile, ra);
    // keys per thread (count <= 8 * 256, checked on the host); unconditional
    // loads (index clamped), so they are all in flight at once
    constexpr int kUnroll = 8;
    unsigned long long kv[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int i = threadIdx.x + kGemvThreads * u;
      kv[u] = keys[min(i, fin.count - 1)];
    }
    // the tile's and the keys' loads need only preloaded arguments: keep them
    // ahead of the wait for the others
    __builtin_amdgcn_sched_barrier(0);
    act.issue_norm(norm_w, K);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if ((int)threadIdx.x + kGemvThreads * u >= fin.count) kv[u] = 0ull;
    const bool recorder = blockIdx.x == 0;
    int st[4] = {0, 0, 0, 0};
    if (recorder && fin.step != nullptr) {
      st[0] = fin.step[0];
      st[1] = fin.step[1];
      st[2] = fin.step[2];
      st[3] = fin.step[3];
    }
    const int at = recorder && fin.history != nullptr ? fin.history_len[0] : 0;
    const int p = st[0] + 1;
    const bool rows = recorder && fin.rope_rows != nullptr && fin.step != nullptr && p < fin.cap &&
                      (int)threadIdx.x < fin.head_dim;
    uint16_t cs = 0, sn = 0;
    if (rows) {
      cs = fin.cos_table[(size_t)p * fin.head_dim + threadIdx.x];
      sn = fin.sin_table[(size_t)p * fin.head_dim + threadIdx.x];
    }
    unsigned long long best = 0;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) best = max_u64(best, kv[u]);
    best = wave_max_u64(best);
    __shared__ unsigned long long s_best[kGemvThreads / 64];
    if (lane == 0) s_best[wave] = best;
    __syncthreads();
    best = max_u64(max_u64(s_best[0], s_best[1]), max_u64(s_best[2], s_best[3]));
    const long long token = argmax_key_index(best);
    const bool ok = token >= 0 && token < fin.embed_rows;
    act.issue_x(x + (size_t)(ok ? token : 0) * K, K, !ok);
    if (recorder) {
      if (threadIdx.x == 0) {
        fin.token_out[0] = token;
        if (fin.history != nullptr) {
          fin.history[at] = token;
          fin.history_len[0] = at + 1;
        }
        if (fin.step != nullptr) {
          fin.step[0] = st[0] + 1;
          fin.step[1] = st[1] + 1;
          fin.step[2] = st[2] + 1 == fin.cap ? 0 : st[2] + 1;
          fin.step[3] = st[3] + 1 == fin.cap ? 0 : st[3] + 1;
        }
        if (!ok && fin.error != nullptr) fin.error[0] = 1;
      }
      if (rows) {
        fin.rope_rows[threadIdx.x] = cs;
        fin.rope_rows[fin.head_dim + threadIdx.x] = sn;
      }
      // the raw row is the step's residual
      uint4* hid = reinterpret_cast<uint4*>(fin.hidden_out);
#pragma unroll
      for (int i = 0; i < (XV > 0 ? XV : 1); ++i) {
        const int v = (int)threadIdx.x + kGemvThreads * i;
        if (v < (K >> 3)) hid[v] = act.xr[i];
      }
    }
    act.finish(eps, K, xp, csum);
    if constexpr (XREG) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
#pragma unroll
        for (int k = 0; k < 4; ++k) xr[j][k] = xp[cidx[j] * 4 + k];
        cr[j] = csum[cidx[j]];
      }
    }
  } else if constexpr (BLOCKX) {
    // every wave takes part in the block's staging barrier, tile or not
    StagedActivation<NORM, (XV > 0 ? XV : 1), false> act;
    act.issue(x, norm_w, K);
    load(tile, ra);
    __builtin_amdgcn_sched_barrier(0);  // x, then the first tile's loads, then the staging
    act.finish(eps, K, xp, csum);
    if constexpr (XREG) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
#pragma unroll
        for (int k = 0; k < 4; ++k) xr[j][k] = xp[cidx[j] * 4 + k];
        cr[j] = csum[cidx[j]];
      }
    }
  }
  if (tile >= tiles) {
    if (ARGMAX && lane == 0) keys[tile] = 0;
    return;
  }
  if constexpr (BLOCKX) {
    // staged above
  } else if constexpr (DIRECT) {
    DirectActivation<LPR, CPL, NORM> act;
    act.issue(x, norm_w, K, li);
    load(tile, ra);
    __builtin_amdgcn_sched_barrier(0);  // x, then every load of the first tile, then the math
    act.finish(eps, K, li, xr, cr);
  } else {
    StagedActivation<NORM, (XV > 0 ? XV : 1), true> act;
    act.issue(x, norm_w, K);
    load(tile, ra);
    // Keep every load of the first tile ahead of the staging code: the
    // scheduler otherwise sinks some of them behind the wait for x, which costs
    // a memory round trip per wave and leaves the loop's entry waits
    // conservative.
    __builtin_amdgcn_sched_barrier(0);
    act.finish(eps, K, xp, csum);
    if (XREG) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
#pragma unroll
        for (int k = 0; k < 4; ++k) xr[j][k] = xp[cidx[j] * 4 + k];
        cr[j] = csum[cidx[j]];
      }
    }
  }
  // The tile count per wave is uniform, so these branches are scalar.
  if constexpr (DIRECT) {
    // Short outputs: a wave has one or two tiles, so its last tile issues no
    // (redundant) prefetch - the wave would otherwise wait for it at exit.
    while (true) {
      if (tile + total_waves >= tiles) {
        consume(tile, ra);
        break;
      }
      load(tile + total_waves, rb);
      consume(tile, ra);
      tile += total_waves;
      if (tile + total_waves >= tiles) {
        consume(tile, rb);
        break;
      }
      load(tile + total_waves, ra);
      consume(tile, rb);
      tile += total_waves;
    }
  } else {
    // Long outputs: many tiles per wave. The trip count is computed up front
    // (uniform), so the loop has one exit and no branch between a load and its
    // use; the prefetch is unconditional (index clamped), and the one redundant
    // prefetch at the end is not used. A loop with an exit in the middle lets
    // the compiler's wait placement merge a path on which the other register
    // set is still in flight into the loop head, which then waits for every
    // outstanding load before issuing the next prefetch.
    // The scheduling barriers keep each prefetch ahead of the math on the
    // other set (the scheduler would otherwise start the math first, and the
    // prefetch would wait behind the current set's loads).
    // (Measured and not kept: both register sets loaded before the x staging,
    // reloads clamped to the wave's own last tile - 0.7-1.4 us slower on every
    // Llama-8B layer projection and the Qwen LM head.)
    const int mine = (tiles - tile + total_waves - 1) / total_waves;
    for (int i = 0; i + 2 <= mine; i += 2) {
      load(tile + total_waves, rb);
      __builtin_amdgcn_sched_barrier(0);
      consume(tile, ra);
      load(tile + 2 * total_waves, ra);
      __builtin_amdgcn_sched_barrier(0);
      consume(tile + total_waves, rb);
      tile += 2 * total_waves;
    }
    if (mine & 1) consume(tile, ra);
  }
  if (ARGMAX) {
    best = wave_max_u64(best);
    if (lane == 0) keys[blockIdx.x * waves_per_block + wave] = best;
  }
}

}  // namespace aoto

// Argument order: what the first loads need comes first, so it arrives in the
// preloaded SGPRs (the code object is built with kernel-argument preloading,
// 14 dwords on gfx950) instead of behind a scalar load from the argument
// buffer: the weights, x, the norm weight, the shape, then the bias element.
#define AOTO_GEMV_STREAM_KERNEL_X(NAME, LPR, CPL, XV, XREG, NORM, PAIRED, BIAS, ARGMAX, BLOCKX)       \
  extern "C" __global__ __launch_bounds__(aoto::kGemvThreads) void NAME(                                 \
      const uint4* words, const uint16_t* scales, const uint16_t* x, const uint16_t* norm_w, int K,      \
      int N, int group_shift, int waves_per_block, const uint16_t* bias, const uint4* up_words,          \
      const uint16_t* up_scales, float eps, float alpha, float beta, uint16_t* y,                        \
      unsigned long long* keys) {                                                                        \
    aoto::w4_gemv_stream_body<LPR, CPL, XV, XREG, NORM, PAIRED, BIAS, ARGMAX, BLOCKX>(                   \
        x, words, scales, up_words, up_scales, norm_w, eps, bias, alpha, beta, y, K, N, group_shift,     \
        waves_per_block, keys);                                                                          \
  }
#define AOTO_GEMV_STREAM_KERNEL(NAME, LPR, CPL, XV, XREG, NORM, PAIRED, BIAS, ARGMAX)                   \
  AOTO_GEMV_STREAM_KERNEL_X(NAME, LPR, CPL, XV, XREG, NORM, PAIRED, BIAS, ARGMAX, false)

#define AOTO_GEMV_STREAM_INSTANCE(LPR, CPL, XV, XREG, NORM, PAIRED, BIAS)                                \
  AOTO_GEMV_STREAM_KERNEL(aoto_w4_gemv_s##LPR##x##CPL##_n##NORM##_p##PAIRED##_b##BIAS, LPR, CPL, XV,     \
                          XREG, NORM, PAIRED, BIAS, false)

// The decode variants a decoder layer uses: q/k/v (norm, +bias or not), o and
// down (+residual), paired gate/up (norm), LM head (norm), plain.
// Single-projection variants (q/k/v with or without bias, o/down residual, LM
// head, plain) and the paired gate/up variants of one lane layout.
#define AOTO_GEMV_STREAM_SINGLE(LPR, CPL, XV, XREG)          \
  AOTO_GEMV_STREAM_INSTANCE(LPR, CPL, XV, XREG, 1, 0, 1)    \
  AOTO_GEMV_STREAM_INSTANCE(LPR, CPL, XV, XREG, 1, 0, 0)    \
  AOTO_GEMV_STREAM_INSTANCE(LPR, CPL, XV, XREG, 0, 0, 1)    \
  AOTO_GEMV_STREAM_INSTANCE(LPR, CPL, XV, XREG, 0, 0, 0)
#define AOTO_GEMV_STREAM_PAIRED(LPR, CPL, XV, XREG)          \
  AOTO_GEMV_STREAM_INSTANCE(LPR, CPL, XV, XREG, 1, 1, 0)    \
  AOTO_GEMV_STREAM_INSTANCE(LPR, CPL, XV, XREG, 0, 1, 0)
// LM head with the greedy-argmax partial keys (with or without the final norm).
#define AOTO_GEMV_STREAM_ARGMAX(LPR, CPL, XV, XREG)                                                      \
  AOTO_GEMV_STREAM_KERNEL(aoto_w4_gemv_s##LPR##x##CPL##_n1_argmax, LPR, CPL, XV, XREG, 1, 0, 0, true)  \
  AOTO_GEMV_STREAM_KERNEL(aoto_w4_gemv_s##LPR##x##CPL##_n0_argmax, LPR, CPL, XV, XREG, 0, 0, 0, true)
// Block-staged single projection with the greedy loop's argmax finish in its
// prologue: aoto_w4_gemv_x{LPR}x{CPL}_n{NORM}_b{BIAS}_finish. What the first
// tile's and the keys' loads need comes first, within the 14 preloaded argument
// dwords: keys, weights, scales, embedding table, K, N, shape = group_shift |
// waves_per_block << 4 | key count << 12, bias.
#define AOTO_GEMV_STREAM_FINISH_KERNEL(LPR, CPL, XV, NORM, BIAS)                                          \
  extern "C" __global__ __launch_bounds__(aoto::kGemvThreads) void                                       \
      aoto_w4_gemv_x##LPR##x##CPL##_n##NORM##_b##BIAS##_finish(                                          \
          unsigned long long* keys, const uint4* words, const uint16_t* scales, const uint16_t* embed,   \
          int K, int N, int shape, const uint16_t* bias, const uint16_t* norm_w, float eps, float alpha,  \
          float beta, uint16_t* y, aoto::GemvFinishArgs fin) {                                            \
    aoto::GemvFinishArgs f = fin;                                                                        \
    f.count = (int)((unsigned)shape >> 12);                                                              \
    aoto::w4_gemv_stream_body<LPR, CPL, XV, true, NORM, false, BIAS, false, true, true>(                 \
        embed, words, scales, nullptr, nullptr, norm_w, eps, bias, alpha, beta, y, K, N, shape & 0xF,    \
        (shape >> 4) & 0xFF, keys, f);                                                                   \
  }
// Block-staged forms (x shared by the block's 4 waves) for long reductions:
// names aoto_w4_gemv_x{LPR}x{CPL}_n*_p*_b*. XREG: each lane then copies its
// chunks of x into registers (single projections; the paired form, with two
// weight sets in flight, keeps reading x from LDS).
#define AOTO_GEMV_STREAM_BLOCKX_INSTANCE(LPR, CPL, XV, XREG, NORM, PAIRED, BIAS)                         \
  AOTO_GEMV_STREAM_KERNEL_X(aoto_w4_gemv_x##LPR##x##CPL##_n##NORM##_p##PAIRED##_b##BIAS, LPR, CPL, XV,   \
                            XREG, NORM, PAIRED, BIAS, false, true)
#define AOTO_GEMV_STREAM_BLOCKX_SINGLE(LPR, CPL, XV)                \
  AOTO_GEMV_STREAM_BLOCKX_INSTANCE(LPR, CPL, XV, true, 1, 0, 1)    \
  AOTO_GEMV_STREAM_BLOCKX_INSTANCE(LPR, CPL, XV, true, 1, 0, 0)    \
  AOTO_GEMV_STREAM_BLOCKX_INSTANCE(LPR, CPL, XV, true, 0, 0, 1)    \
  AOTO_GEMV_STREAM_BLOCKX_INSTANCE(LPR, CPL, XV, true, 0, 0, 0)
#define AOTO_GEMV_STREAM_BLOCKX_PAIRED(LPR, CPL, XV)                 \
  AOTO_GEMV_STREAM_BLOCKX_INSTANCE(LPR, CPL, XV, false, 1, 1, 0)    \
  AOTO_GEMV_STREAM_BLOCKX_INSTANCE(LPR, CPL, XV, false, 0, 1, 0)
