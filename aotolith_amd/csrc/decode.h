// Decode-step kernels other than the GEMV: the fused RoPE + KV-cache append,
// single-query GQA attention, the embedding gather and the greedy argmax.
//
// Cache layout (the reference's cache ABI, models/decoder.py:554-561):
//   cache[L][2][B][Hkv][cap][D] bf16, pair 0 = keys, pair 1 = values.
// A projection row is [B][W] bf16 with q at query_start, k at key_start and v at
// value_start (W = (Hq + 2 Hkv) D for the packed q/k/v projection).
#pragma once

#include "common.h"

namespace aoto {

// x * cos + rotate_half(x) * sin for one element, f32, one rounding
// (codegen/kv_cache.py:144-159: the partner of column d is d +- D/2 and the
// first half takes it negated).
AOTO_DEVICE float rope_value(const uint16_t* __restrict__ head, const uint16_t* __restrict__ cos_row,
                             const uint16_t* __restrict__ sin_row, int d, int half) {
  const float x = bf16_to_f32(head[d]);
  const float partner = d < half ? -bf16_to_f32(head[d + half]) : bf16_to_f32(head[d - half]);
  return x * bf16_to_f32(cos_row[d]) + partner * bf16_to_f32(sin_row[d]);
}

// Rotate the step's q and k out of the projection row and write one layer's
// next cache window.
//
// * `mode == 0` (roll, the reference's functional op): pair_out[p][b][h][s] =
//   pair_in[p][b][h][s + 1] for s < cap - 1 and the new (k_rot, v) at slot
//   cap - 1. pair_in / pair_out are one layer's [2][B][Hkv][cap][D] windows and
//   must not overlap.
// * `mode == 1` (ring): (k_rot, v) is written in place at slot `slot` of
//   pair_out; nothing else moves (pair_in is unused).
// With `step` non-null the position and slot come from device memory
// (step[0] = position, step[3] = slot), so a captured decode step replays
// without host updates. q_out is [B][Hq][D]. Work items: B*Hq*D query elements, B*Hkv*D key and value
// elements, then (roll only) the copy of the 2*B*Hkv*(cap-1)*D window, 8
// elements per thread.
extern "C" __global__ __launch_bounds__(256) void aoto_rope_kv_append(
    const uint16_t* __restrict__ row, int row_width, const uint16_t* __restrict__ cos_table,
    const uint16_t* __restrict__ sin_table, int position, const uint16_t* __restrict__ pair_in,
    uint16_t* __restrict__ pair_out, uint16_t* __restrict__ q_out, int batch, int query_heads,
    int kv_heads, int cap, int D, int query_start, int key_start, int value_start, int mode, int slot,
    const int* __restrict__ step) {
  const long long tid = (long long)blockIdx.x * 256 + threadIdx.x;
  const int half = D >> 1;
  if (step != nullptr) {
    position = step[0];
    slot = step[3];
  }
  const uint16_t* cos_row = cos_table + (size_t)position * D;
  const uint16_t* sin_row = sin_table + (size_t)position * D;
  const long long q_items = (long long)batch * query_heads * D;
  const long long kv_items = (long long)batch * kv_heads * D;
  if (tid < q_items) {
    const int d = (int)(tid % D);
    const long long bh = tid / D;
    const int b = (int)(bh / query_heads), h = (int)(bh % query_heads);
    const uint16_t* head = row + (size_t)b * row_width + query_start + (size_t)h * D;
    q_out[tid] = (uint16_t)f32_to_bf16(rope_value(head, cos_row, sin_row, d, half));
    return;
  }
  long long t = tid - q_items;
  const size_t head_stride = (size_t)cap * D;
  const size_t pair_stride = (size_t)batch * kv_heads * head_stride;
  const int last = mode == 0 ? cap - 1 : slot;
  if (t < kv_items) {
    const int d = (int)(t % D);
    const long long bh = t / D;
    const int b = (int)(bh / kv_heads), h = (int)(bh % kv_heads);
    const uint16_t* khead = row + (size_t)b * row_width + key_start + (size_t)h * D;
    const uint16_t* vhead = row + (size_t)b * row_width + value_start + (size_t)h * D;
    const size_t dst = ((size_t)b * kv_heads + h) * head_stride + (size_t)last * D + d;
    pair_out[dst] = (uint16_t)f32_to_bf16(rope_value(khead, cos_row, sin_row, d, half));
    pair_out[pair_stride + dst] = vhead[d];
    return;
  }
  if (mode != 0) return;
  t -= kv_items;
  // Roll: 8-element vectors of the 2*B*Hkv heads' first cap-1 output slots.
  const int vec_per_row = D >> 3;
  const long long per_head = (long long)(cap - 1) * vec_per_row;
  const long long total = 2LL * batch * kv_heads * per_head;
  if (t >= total) return;
  const long long head_index = t / per_head;
  const long long within = t - head_index * per_head;
  const size_t dst = (size_t)head_index * head_stride + (size_t)within * 8;
  reinterpret_cast<uint4*>(pair_out + dst)[0] = reinterpret_cast<const uint4*>(pair_in + dst + D)[0];
}

// Single-query GQA attention over one layer's cache window (codegen/attention.py:
// 447-656 semantics; runtime/mlx_ops/attention.py:89-122):
//   out[b][h] = softmax(scale * q[b][h] . K[b][h/G]^T, keep) V[b][h/G]
// scores and softmax in f32, fully masked heads give 0, one rounding at the end.
//
// Which key slots are kept: with `mask` non-null, mask[b*mask_batch_stride + s]
// != 0; otherwise the slots whose logical index (s - ring_offset) mod cap is at
// least cap - valid (the last `valid` slots of the reference's rolled window when
// ring_offset == 0; a ring buffer rotated by ring_offset otherwise).
//
// FUSED (the ring-buffer decode step): q is not an input. The block rotates its
// query head and its kv head's new key straight out of the projection row
// (`row`, table row `position`), takes the new value from the row, uses both
// for slot `slot` instead of the cache contents, and the first query head of
// each kv group, in the split whose key range holds `slot`, stores the new
// (k_rot, v) there. This folds the rope_kv_cache_append node into the launch.
// With `step` non-null, {position, valid, ring_offset, slot} come from the
// device step state of a captured decode loop.
//
// Grid (splits, B*Hq); 256 threads; one query head per block, keys
// [split*chunk, min(cap, (split+1)*chunk)). The decode window is tiny, so the
// design minimizes dependent steps rather than bytes: every key row is one
// lane's (D/64 lanes per key, 64 dims each, q in registers), so a score needs
// no cross-lane reduction; P.V gives each thread a pair of dims and a strided
// subset of keys. All of a block's K and V loads are independent and issued
// together. One split writes the output; several write (max, sum, acc[D])
// records that aoto_decode_attention_merge combines in a second launch.
template <int D, bool FUSED>
__device__ void decode_attention_body(const uint16_t* __restrict__ q, const uint16_t* __restrict__ row,
                                      int row_width, int query_start, int key_start, int value_start,
                                      const uint16_t* __restrict__ cos_table, const uint16_t* __restrict__ sin_table,
                                      uint16_t* __restrict__ kbase, uint16_t* __restrict__ vbase,
                                      long long kv_batch_stride, long long kv_head_stride,
                                      const uint8_t* __restrict__ mask, int mask_batch_stride, int valid,
                                      int ring_offset, int position, int slot, int cap, int query_heads,
                                      int kv_heads, float scale, int chunk, float* __restrict__ partials,
                                      const int* __restrict__ step, const uint16_t* __restrict__ rope_rows,
                                      uint16_t* __restrict__ out) {
  constexpr int THREADS = 256;
  constexpr int LPK = D / 64;             // lanes per key (64 dims each)
  constexpr int KPP = THREADS / LPK;      // keys per block (one key row per D/64 lanes)
  constexpr int PAIRS = D / 2;            // bf16 pairs per row
  constexpr int KG = THREADS / PAIRS;     // key groups in P.V
  constexpr int VPT = KPP / KG;           // value pairs per thread (all loaded up front)
  __shared__ __attribute__((aligned(16))) float s_p[KPP];
  __shared__ float s_red[THREADS / 64];
  __shared__ float s_acc[KG][D];
  __shared__ __attribute__((aligned(16))) float s_q[D];
  __shared__ __attribute__((aligned(16))) uint16_t s_knew[D];
  __shared__ __attribute__((aligned(16))) uint16_t s_vnew[D];

  const int split = blockIdx.x;
  const int splits = gridDim.x;
  const int bh = blockIdx.y;
  const int b = bh / query_heads, h = bh % query_heads;
  const int group = query_heads / kv_heads;
  const int kvh = h / group;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int s0 = split * chunk;
  const int n = max(0, min(cap, s0 + chunk) - s0);  // <= KPP, checked on the host
  const int sub = threadIdx.x % LPK;      // which 64 dims of a key row
  const int kl = threadIdx.x / LPK;       // this thread's key
  const int d2 = threadIdx.x % PAIRS;     // P.V: this thread's dim pair
  const int kg = threadIdx.x / PAIRS;     // P.V: keys kg, kg + KG, ...

  uint16_t* kh = kbase + (size_t)b * kv_batch_stride + (size_t)kvh * kv_head_stride;
  uint16_t* vh = vbase + (size_t)b * kv_batch_stride + (size_t)kvh * kv_head_stride;

  // Every K and V row of the block is loaded first: those addresses do not
  // depend on the device step state, whose read (and the RoPE table rows it
  // selects) would otherwise hold back every other load by a round trip.
  const int ksl = s0 + min(kl, max(n - 1, 0));
  uint4 kv[8];
  {
    const uint4* kr = reinterpret_cast<const uint4*>(kh + (size_t)ksl * D);
#pragma unroll
    for (int c = 0; c < 8; ++c) kv[c] = kr[sub * 8 + c];
  }
  // P.V work split: thread (kg, d2) owns dims (2*d2, 2*d2+1) of keys
  // [kg*VPT, (kg+1)*VPT), so its probabilities are one contiguous LDS run.
  const int kbase0 = kg * VPT;
  uint32_t vv[VPT];
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const int sl = s0 + min(kbase0 + u, max(n - 1, 0));
    vv[u] = reinterpret_cast<const uint32_t*>(vh + (size_t)sl * D)[d2];
  }
  // The query / new key / new value of this head, and the RoPE rows of the
  // position: from `rope_rows` (cos row, then sin row) when given - no
  // dependence on the step state - else from the tables at the step's position.
  const int d = min((int)threadIdx.x, D - 1);
  uint32_t qx = 0, qp = 0, kx = 0, kp = 0, cs = 0, sn = 0, vx = 0;
  const int half = D / 2;
  const int pd = d < half ? d + half : d - half;
  if (FUSED) {
    const uint16_t* rrow = row + (size_t)b * row_width;
    const uint16_t* qh = rrow + query_start + (size_t)h * D;
    const uint16_t* khh = rrow + key_start + (size_t)kvh * D;
    qx = qh[d];
    qp = qh[pd];
    kx = khh[d];
    kp = khh[pd];
    vx = rrow[value_start + (size_t)kvh * D + d];
    if (rope_rows != nullptr) {
      cs = rope_rows[d];
      sn = rope_rows[D + d];
    }
  } else {
    qx = q[((size_t)b * query_heads + h) * D + d];
  }
  if (step != nullptr) {
    position = step[0];
    valid = step[1];
    ring_offset = step[2];
    slot = step[3];
  }
  if (FUSED && rope_rows == nullptr) {
    cs = cos_table[(size_t)position * D + d];
    sn = sin_table[(size_t)position * D + d];
  }

  // Query (rotated out of the projection row when FUSED) into LDS, f32.
  if (threadIdx.x < D) {
    if (FUSED) {
      const float sign = d < half ? -1.f : 1.f;
      const float c = bf16_to_f32(cs), sv = bf16_to_f32(sn);
      s_q[d] = round_bf16(bf16_to_f32(qx) * c + sign * bf16_to_f32(qp) * sv);
      s_knew[d] = (uint16_t)f32_to_bf16(bf16_to_f32(kx) * c + sign * bf16_to_f32(kp) * sv);
      s_vnew[d] = (uint16_t)vx;
    } else {
      s_q[d] = bf16_to_f32(qx);
    }
  }
  __syncthreads();
  if (FUSED && ksl == slot) {
#pragma unroll
    for (int c = 0; c < 8; ++c) kv[c] = reinterpret_cast<const uint4*>(s_knew)[sub * 8 + c];
  }
  if (FUSED) {
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int sl = s0 + min(kbase0 + u, max(n - 1, 0));
      if (sl == slot) vv[u] = reinterpret_cast<const uint32_t*>(s_vnew)[d2];
    }
  }

  auto kept = [&](int sl) -> bool {
    if (mask != nullptr) return mask[(size_t)b * mask_batch_stride + sl] != 0;
    int logical = sl - ring_offset;
    logical += logical < 0 ? cap : 0;
    return logical >= cap - valid;
  };

  // Score of this thread's key (64 dims per lane).
  float dot = 0.f;
  const float4* qs = reinterpret_cast<const float4*>(s_q + sub * 64);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float4 qa = qs[2 * c], qb = qs[2 * c + 1];
    const uint32_t a[4] = {kv[c].x, kv[c].y, kv[c].z, kv[c].w};
    dot = fmaf(qa.x, bf16_lo(a[0]), dot);
    dot = fmaf(qa.y, bf16_hi(a[0]), dot);
    dot = fmaf(qa.z, bf16_lo(a[1]), dot);
    dot = fmaf(qa.w, bf16_hi(a[1]), dot);
    dot = fmaf(qb.x, bf16_lo(a[2]), dot);
    dot = fmaf(qb.y, bf16_hi(a[2]), dot);
    dot = fmaf(qb.z, bf16_lo(a[3]), dot);
    dot = fmaf(qb.w, bf16_hi(a[3]), dot);
  }
  if (LPK == 2) dot += dpp_move<kDppXor1>(dot);
  float sc = -INFINITY;
  if (kl < n && kept(ksl)) sc = dot * scale;
  if (sub == 0 && kl < n) s_p[kl] = sc;
  const float m = wave_max(sc);
  if (lane == 0) s_red[wave] = m;
  __syncthreads();
  float row_max = s_red[0];
#pragma unroll
  for (int w = 1; w < THREADS / 64; ++w) row_max = fmaxf(row_max, s_red[w]);
  __syncthreads();  // s_red is reused below
  // Probabilities; slots past the range read as 0 in P.V.
  float p_local = 0.f;
  if (threadIdx.x < KPP) {
    if (threadIdx.x < n) {
      const float v = s_p[threadIdx.x];
      p_local = (row_max == -INFINITY || v == -INFINITY) ? 0.f : expf(v - row_max);
    }
    s_p[threadIdx.x] = p_local;
  }
  const float t = wave_sum(p_local);
  if (lane == 0) s_red[wave] = t;
  __syncthreads();
  float row_sum = 0.f;
#pragma unroll
  for (int w = 0; w < THREADS / 64; ++w) row_sum += s_red[w];

  // P.V over this thread's keys and dim pair.
  float a0 = 0.f, a1 = 0.f;
  const float4* pv4 = reinterpret_cast<const float4*>(s_p + kbase0);
#pragma unroll
  for (int u4 = 0; u4 < VPT / 4; ++u4) {
    const float4 pr = pv4[u4];
    const float pp[4] = {pr.x, pr.y, pr.z, pr.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a0 = fmaf(pp[e], bf16_lo(vv[u4 * 4 + e]), a0);
      a1 = fmaf(pp[e], bf16_hi(vv[u4 * 4 + e]), a1);
    }
  }
  s_acc[kg][2 * d2] = a0;
  s_acc[kg][2 * d2 + 1] = a1;
  __syncthreads();
  if (FUSED && h % group == 0 && slot >= s0 && slot < s0 + n && threadIdx.x < D) {
    kh[(size_t)slot * D + threadIdx.x] = s_knew[threadIdx.x];
    vh[(size_t)slot * D + threadIdx.x] = s_vnew[threadIdx.x];
  }
  if (threadIdx.x < D) {
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < KG; ++g) acc += s_acc[g][d];
    if (splits == 1) {
      out[((size_t)b * query_heads + h) * D + d] = (uint16_t)f32_to_bf16(row_sum > 0.f ? acc / row_sum : 0.f);
    } else {
      float* rec = partials + (((size_t)b * query_heads + h) * splits + split) * (D + 2);
      rec[2 + d] = acc;
      if (d == 0) {
        rec[0] = row_max;
        rec[1] = row_sum;
      }
    }
  }
}

// Combine the split records of aoto_decode_attention_*: one block per (b, head),
//   out = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s,  M = max_s m_s; 0 when no key is kept.
// Every load is independent of the others (split s's record is read by thread
// s % 128, then each thread reads its column of all records with an unrolled
// loop), so a merge costs a couple of memory round trips, not one per split.
// splits <= kMergeMaxSplits (checked on the host).
constexpr int kMergeMaxSplits = 1024;
extern "C" __global__ __launch_bounds__(128) void aoto_decode_attention_merge(const float* __restrict__ partials,
                                                                             int splits, int D,
                                                                             uint16_t* __restrict__ out) {
  __shared__ float s_w[kMergeMaxSplits];
  __shared__ float s_red[2];
  const int bh = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float* rec = partials + (size_t)bh * splits * (D + 2);
  float m = -INFINITY;
  for (int s = threadIdx.x; s < splits; s += 128) m = fmaxf(m, rec[(size_t)s * (D + 2)]);
  m = wave_max(m);
  if (lane == 0) s_red[wave] = m;
  __syncthreads();
  const float M = fmaxf(s_red[0], s_red[1]);
  __syncthreads();  // s_red is reused for the denominator
  float den = 0.f;
  for (int s = threadIdx.x; s < splits; s += 128) {
    const float ms = rec[(size_t)s * (D + 2)];
    const float ls = rec[(size_t)s * (D + 2) + 1];
    const float w = (M == -INFINITY || ms == -INFINITY) ? 0.f : expf(ms - M);
    s_w[s] = w;
    den = fmaf(w, ls, den);
  }
  den = wave_sum(den);
  if (lane == 0) s_red[wave] = den;
  __syncthreads();
  den = s_red[0] + s_red[1];
  for (int d = threadIdx.x; d < D; d += 128) {
    float num = 0.f;
#pragma unroll 8
    for (int s = 0; s < splits; ++s) num = fmaf(s_w[s], rec[(size_t)s * (D + 2) + 2 + d], num);
    out[(size_t)bh * D + d] = (uint16_t)f32_to_bf16(den > 0.f ? num / den : 0.f);
  }
}

// Embedding gather: out[i][:] = weight[ids[i]][:] for `count` ids (int64 on
// the device, so a captured decode step reads the token the previous step
// produced). Ids outside [0, vocab) produce a zero row and set *error to 1
// (bounds are checked, never faulted). 8 elements per thread.
extern "C" __global__ __launch_bounds__(256) void aoto_embedding(
    const uint16_t* __restrict__ weight, const long long* __restrict__ ids, int count, int hidden,
    long long vocab, uint16_t* __restrict__ out, int* __restrict__ error) {
  const int vec = hidden >> 3;
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long long)count * vec) return;
  const int i = (int)(t / vec), c = (int)(t % vec);
  const long long id = ids[i];
  uint4 value = make_uint4(0, 0, 0, 0);
  if (id >= 0 && id < vocab) {
    value = reinterpret_cast<const uint4*>(weight + (size_t)id * hidden)[c];
  } else if (error != nullptr) {
    error[0] = 1;
  }
  reinterpret_cast<uint4*>(out + (size_t)i * hidden)[c] = value;
}

// Greedy argmax of `rows` rows of `n` bf16 logits (first index on ties,
// models/decoder.py:1069, 1080). One block of 1024 threads per row; 8 values
// per 16-byte load when the row is 16-byte aligned, scalar otherwise. Writes
// int64 token ids; with `history` non-null also appends the token at
// history[*history_len] and bumps the length (the decode loop's token record).
extern "C" __global__ __launch_bounds__(1024) void aoto_argmax(const uint16_t* __restrict__ logits, int n,
                                                               long long row_stride, long long* __restrict__ out,
                                                               long long* __restrict__ history,
                                                               int* __restrict__ history_len) {
  __shared__ unsigned long long s_best[16];
  const uint16_t* row = logits + (size_t)blockIdx.x * row_stride;
  unsigned long long best = 0;
  const bool vec = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0) && (n % 8 == 0);
  if (vec) {
    const uint4* rv = reinterpret_cast<const uint4*>(row);
    for (int c = threadIdx.x; c < n / 8; c += 1024) {
      const uint4 r = rv[c];
      const uint32_t raw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        best = max_u64(best, argmax_key(raw[j] & 0xFFFFu, c * 8 + 2 * j));
        best = max_u64(best, argmax_key(raw[j] >> 16, c * 8 + 2 * j + 1));
      }
    }
  } else {
    for (int i = threadIdx.x; i < n; i += 1024) best = max_u64(best, argmax_key(row[i], i));
  }
  best = wave_max_u64(best);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) s_best[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long m = 0;
    for (int w = 0; w < 16; ++w) m = max_u64(m, s_best[w]);
    const long long token = argmax_key_index(m);
    out[blockIdx.x] = token;
    if (history != nullptr && gridDim.x == 1) {
      const int at = history_len[0];
      history[at] = token;
      history_len[0] = at + 1;
    }
  }
}

// Finish of the fused LM-head argmax: reduce the `count` partial keys written by
// an *_argmax streaming GEMV to the greedy token (first index on ties), store it
// at token_out[0], and then, each when its pointer is non-null:
//   history   append the token at history[*history_len], bump the length;
//   step      advance the decode-loop step state {position, valid, ring_offset,
//             slot} by one token (as aoto_step_advance);
//   embed     gather embedding row `token` (bf16 [embed_rows, hidden]) into
//             hidden_out - the next decode step's input - or zeros and
//             error[0] = 1 if the token is not a row of the table.
//   rope_rows (with step) the cos and sin rows of the advanced position
//             (tables [cap, D]) - the next step's RoPE rows, so its attention
//             kernels need not read the step state before loading them.
// One block of 256 threads; hidden % 8 == 0.
extern "C" __global__ __launch_bounds__(256) void aoto_argmax_finish(
    const unsigned long long* __restrict__ keys, int count, long long* __restrict__ token_out,
    long long* __restrict__ history, int* __restrict__ history_len, int* __restrict__ step, int cap,
    const uint16_t* __restrict__ embed, long long embed_rows, int hidden, uint16_t* __restrict__ hidden_out,
    int* __restrict__ error, const uint16_t* __restrict__ cos_table, const uint16_t* __restrict__ sin_table,
    int head_dim, uint16_t* __restrict__ rope_rows) {
  __shared__ unsigned long long s_best[4];
  __shared__ long long s_token;
  __shared__ int s_position;
  unsigned long long best = 0;
  for (int i = threadIdx.x; i < count; i += 256) best = max_u64(best, keys[i]);
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned long long m = max_u64(max_u64(s_best[0], s_best[1]), max_u64(s_best[2], s_best[3]));
    const long long token = argmax_key_index(m);
    token_out[0] = token;
    if (history != nullptr) {
      const int at = history_len[0];
      history[at] = token;
      history_len[0] = at + 1;
    }
    if (step != nullptr) {
      s_position = step[0] + 1;
      step[0] += 1;
      step[1] += 1;
      step[2] = step[2] + 1 == cap ? 0 : step[2] + 1;
      step[3] = step[3] + 1 == cap ? 0 : step[3] + 1;
    }
    s_token = token;
  }
  __syncthreads();
  if (rope_rows != nullptr && step != nullptr) {
    // a position past the tables (the step after the last) keeps the old rows
    const int p = s_position;
    if (p < cap) {
      for (int i = threadIdx.x; i < head_dim; i += 256) {
        rope_rows[i] = cos_table[(size_t)p * head_dim + i];
        rope_rows[head_dim + i] = sin_table[(size_t)p * head_dim + i];
      }
    }
  }
  if (embed == nullptr) return;
  const long long token = s_token;
  const bool ok = token >= 0 && token < embed_rows;
  if (!ok && threadIdx.x == 0 && error != nullptr) error[0] = 1;
  const uint4* src = reinterpret_cast<const uint4*>(embed + (size_t)(ok ? token : 0) * hidden);
  uint4* dst = reinterpret_cast<uint4*>(hidden_out);
  for (int c = threadIdx.x; c < (hidden >> 3); c += 256) dst[c] = ok ? src[c] : make_uint4(0, 0, 0, 0);
}

// Advance the decode-loop step state by one token: position and valid length
// grow by one, the ring offset and the next write slot move one slot on
// (state = {position, valid, ring_offset, slot}). One thread.
extern "C" __global__ void aoto_step_advance(int* __restrict__ state, int cap) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  state[0] += 1;
  state[1] += 1;
  state[2] = state[2] + 1 == cap ? 0 : state[2] + 1;
  state[3] = state[3] + 1 == cap ? 0 : state[3] + 1;
}

}  // namespace aoto

#define AOTO_DECODE_ATTENTION_INSTANCE(D)                                                                \
  extern "C" __global__ __launch_bounds__(256) void aoto_decode_attention_d##D(                         \
      const uint16_t* q, uint16_t* kbase, uint16_t* vbase, long long kv_batch_stride,                    \
      long long kv_head_stride, const uint8_t* mask, int mask_batch_stride, int valid, int ring_offset,  \
      int cap, int query_heads, int kv_heads, float scale, int chunk, float* partials, const int* step,  \
      uint16_t* out) {                                                                                   \
    aoto::decode_attention_body<D, false>(q, nullptr, 0, 0, 0, 0, nullptr, nullptr, kbase, vbase,        \
                                          kv_batch_stride, kv_head_stride, mask, mask_batch_stride,      \
                                          valid, ring_offset, 0, -1, cap, query_heads, kv_heads, scale,  \
                                          chunk, partials, step, nullptr, out);                          \
  }                                                                                                      \
  extern "C" __global__ __launch_bounds__(256) void aoto_decode_rope_attention_d##D(                    \
      const uint16_t* row, int row_width, int query_start, int key_start, int value_start,               \
      const uint16_t* cos_table, const uint16_t* sin_table, uint16_t* kbase, uint16_t* vbase,            \
      long long kv_batch_stride, long long kv_head_stride, int valid, int ring_offset, int position,     \
      int slot, int cap, int query_heads, int kv_heads, float scale, int chunk, float* partials,          \
      const int* step, const uint16_t* rope_rows, uint16_t* out) {                                       \
    aoto::decode_attention_body<D, true>(nullptr, row, row_width, query_start, key_start, value_start,   \
                                         cos_table, sin_table, kbase, vbase, kv_batch_stride,            \
                                         kv_head_stride, nullptr, 0, valid, ring_offset, position, slot, \
                                         cap, query_heads, kv_heads, scale, chunk, partials, step,       \
                                         rope_rows, out);                                                \
  }
