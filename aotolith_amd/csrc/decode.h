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
// Grid (splits, B*Hq); WAVES waves per block; one query head per block, keys
// [split*chunk, min(cap, (split+1)*chunk)), chunk <= WAVES * J * 512 / D (each
// wave issues J wave loads of K and J of V; the host picks the instance whose
// J fits the chunk with no idle loads). The window is tiny, so the design
// minimizes dependent steps and keeps every load coalesced:
// * a key row is D/8 lanes, 16 bytes (8 dims) each, so one wave load reads
//   64/(D/8) consecutive rows - 1 KB contiguous - of K or V;
// * wave w owns a contiguous run of the split's keys; its K and V chunks, the
//   query (and, FUSED, the new key/value and RoPE rows) are all loaded up
//   front, the small loads first so the RoPE can start while K and V land;
// * a score is 4 bf16 dot2 per lane and a DPP sum over the row's D/8 lanes;
//   each wave keeps its own softmax (max m_w, sum l_w, unnormalized P.V over its
//   keys, 8 dims per lane; at D = 64 the two keys of a 16-lane row are summed
//   with one DPP move first), so the block meets at one barrier, where D
//   threads combine the waves' records (the same rescaling the split merge
//   uses).
// ROWS: the RoPE rows come from `rope_rows` (no dependence on the step state);
// otherwise from the tables at the position. One split writes the output;
// several write (max, sum, acc[D]) records that aoto_decode_attention_merge
// combines in a second launch.
template <int D, int WAVES, int J, bool FUSED, bool ROWS>
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
  constexpr int LPK = D / 8;                    // lanes per key row (8 dims each)
  constexpr int KPI = 64 / LPK;                 // key rows per wave load
  constexpr int HALF_LANES = LPK / 2;           // lanes holding the first half of a row
  constexpr int SLOTS = 4 * LPK;                // P.V records per wave (4 key lanes per dim)
  static_assert(KPI == 4 || KPI == 8, "D = 64 or 128");
  __shared__ __attribute__((aligned(16))) float s_acc[WAVES][SLOTS][8];
  __shared__ float s_m[WAVES], s_l[WAVES];

  const int split = blockIdx.x;
  const int splits = gridDim.x;
  const int bh = blockIdx.y;
  const int b = bh / query_heads, h = bh % query_heads;
  const int group = query_heads / kv_heads;
  const int kvh = h / group;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPK;                   // dims [8*sub, 8*sub + 8)
  const int kin = lane / LPK;                   // key within a wave load
  const int s0 = split * chunk;
  const int n = max(0, min(cap, s0 + chunk) - s0);  // <= KPI * J * WAVES, checked on the host
  const int loads = (n + WAVES * KPI - 1) / (WAVES * KPI);  // wave loads per wave, <= J
  const int wfirst = wave * loads * KPI;        // this wave's first key (split-relative)

  uint16_t* kh = kbase + (size_t)b * kv_batch_stride + (size_t)kvh * kv_head_stride;
  uint16_t* vh = vbase + (size_t)b * kv_batch_stride + (size_t)kvh * kv_head_stride;

  // Small loads first: the query chunk (and its RoPE partner), the new key /
  // value chunks and the RoPE rows (from `rope_rows` when given, so nothing
  // waits on the device step state), then K and V.
  const int psub = (sub + HALF_LANES) % LPK;    // partner chunk: dims d +- D/2
  uint4 qc, qpc = make_uint4(0, 0, 0, 0), kc = qpc, kpc = qpc, vc = qpc, cc = qpc, sc = qpc;
  if (FUSED) {
    const uint16_t* rrow = row + (size_t)b * row_width;
    const uint4* qh = reinterpret_cast<const uint4*>(rrow + query_start + (size_t)h * D);
    const uint4* khh = reinterpret_cast<const uint4*>(rrow + key_start + (size_t)kvh * D);
    qc = qh[sub];
    qpc = qh[psub];
    kc = khh[sub];
    kpc = khh[psub];
    vc = reinterpret_cast<const uint4*>(rrow + value_start + (size_t)kvh * D)[sub];
    if (ROWS) {
      cc = reinterpret_cast<const uint4*>(rope_rows)[sub];
      sc = reinterpret_cast<const uint4*>(rope_rows + D)[sub];
    }
  } else {
    qc = reinterpret_cast<const uint4*>(q + ((size_t)b * query_heads + h) * D)[sub];
  }
  // Keep these ahead of K and V: loads complete in issue order, so the RoPE's
  // wait then leaves K and V in flight.
  __builtin_amdgcn_sched_barrier(0);
  // K then V chunks of this wave's keys (the last row repeats past n). All J
  // loads are issued, with no branch between them, so the wait before the
  // RoPE covers only the small loads; loads past `loads` are never used.
  uint4 kq[J], vq[J];
  const int last = max(n - 1, 0);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int key = s0 + min(wfirst + j * KPI + kin, last);
    kq[j] = reinterpret_cast<const uint4*>(kh + (size_t)key * D)[sub];
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int key = s0 + min(wfirst + j * KPI + kin, last);
    vq[j] = reinterpret_cast<const uint4*>(vh + (size_t)key * D)[sub];
  }
  __builtin_amdgcn_sched_barrier(0);

  if (step != nullptr) {
    position = step[0];
    valid = step[1];
    ring_offset = step[2];
    slot = step[3];
  }
  if (FUSED && !ROWS) {
    cc = reinterpret_cast<const uint4*>(cos_table + (size_t)position * D)[sub];
    sc = reinterpret_cast<const uint4*>(sin_table + (size_t)position * D)[sub];
  }
  // RoPE of the query (and new key) for this lane's 8 dims, f32, one rounding
  // to bf16 (codegen/kv_cache.py:144-159), packed as bf16 pairs for dot2.
  uint32_t qw[4], knew[4];
  {
    const uint32_t qa[4] = {qc.x, qc.y, qc.z, qc.w};
    if (FUSED) {
      const uint32_t qp[4] = {qpc.x, qpc.y, qpc.z, qpc.w}, ka[4] = {kc.x, kc.y, kc.z, kc.w};
      const uint32_t kp[4] = {kpc.x, kpc.y, kpc.z, kpc.w};
      const uint32_t ca[4] = {cc.x, cc.y, cc.z, cc.w}, sa[4] = {sc.x, sc.y, sc.z, sc.w};
      const float sign = sub < HALF_LANES ? -1.f : 1.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float c0 = bf16_lo(ca[i]), c1 = bf16_hi(ca[i]), s0v = bf16_lo(sa[i]), s1v = bf16_hi(sa[i]);
        qw[i] = pack_bf16x2(bf16_lo(qa[i]) * c0 + sign * bf16_lo(qp[i]) * s0v,
                            bf16_hi(qa[i]) * c1 + sign * bf16_hi(qp[i]) * s1v);
        knew[i] = pack_bf16x2(bf16_lo(ka[i]) * c0 + sign * bf16_lo(kp[i]) * s0v,
                              bf16_hi(ka[i]) * c1 + sign * bf16_hi(kp[i]) * s1v);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) qw[i] = qa[i];
    }
  }

  auto kept = [&](int sl) -> bool {
    if (mask != nullptr) return mask[(size_t)b * mask_batch_stride + sl] != 0;
    int logical = sl - ring_offset;
    logical += logical < 0 ? cap : 0;
    return logical >= cap - valid;
  };

  // Scores of this wave's keys; the slot being written uses the new key.
  float score[J];
  float wmax = -INFINITY;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    score[j] = -INFINITY;
    if (j < loads) {
      const int rel = wfirst + j * KPI + kin;
      const int key = s0 + min(rel, last);
      uint4 k = kq[j];
      if (FUSED) {
        const bool mine = key == slot;
        k.x = mine ? knew[0] : k.x;
        k.y = mine ? knew[1] : k.y;
        k.z = mine ? knew[2] : k.z;
        k.w = mine ? knew[3] : k.w;
      }
      float dot = dot2_bf16(k.x, qw[0], 0.f);
      dot = dot2_bf16(k.y, qw[1], dot);
      dot = dot2_bf16(k.z, qw[2], dot);
      dot = dot2_bf16(k.w, qw[3], dot);
      dot = group_sum<LPK>(dot);
      score[j] = (rel < n && kept(key)) ? dot * scale : -INFINITY;
      wmax = fmaxf(wmax, score[j]);
    }
  }
  const float m = wave_max(wmax);

  // This wave's probabilities, their sum and its P.V over 8 dims per lane.
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (j < loads) {
      const float pj = (m == -INFINITY || score[j] == -INFINITY) ? 0.f : expf(score[j] - m);
      lsum += pj;
      uint4 v = vq[j];
      if (FUSED) {
        const int key = s0 + min(wfirst + j * KPI + kin, last);
        const bool mine = key == slot;
        v.x = mine ? vc.x : v.x;
        v.y = mine ? vc.y : v.y;
        v.z = mine ? vc.z : v.z;
        v.w = mine ? vc.w : v.w;
      }
      const uint32_t va[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = fmaf(pj, bf16_lo(va[i]), acc[2 * i]);
        acc[2 * i + 1] = fmaf(pj, bf16_hi(va[i]), acc[2 * i + 1]);
      }
    }
  }
  // Each key's probability sits in all LPK lanes of its row: count it once.
  const float l = wave_sum(sub == 0 ? lsum : 0.f);
  // Four records per dim: at D = 64 (two key rows per 16-lane row) the rows'
  // pairs are summed first (row_ror:8, i.e. lane ^ 8).
  if (KPI == 8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += dpp_move<0x128>(acc[e]);
  }
  if (KPI == 4 || (lane & 8) == 0) {
    const int rec = (lane >> 4) * LPK + sub;
    reinterpret_cast<float4*>(s_acc[wave][rec])[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    reinterpret_cast<float4*>(s_acc[wave][rec])[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  if (lane == 0) {
    s_m[wave] = m;
    s_l[wave] = l;
  }
  // The first query head of each kv group stores the new (k_rot, v) row.
  if (FUSED && h % group == 0) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int rel = wfirst + j * KPI + kin;
      if (j < loads && rel < n && s0 + rel == slot) {
        reinterpret_cast<uint4*>(kh + (size_t)slot * D)[sub] = make_uint4(knew[0], knew[1], knew[2], knew[3]);
        reinterpret_cast<uint4*>(vh + (size_t)slot * D)[sub] = vc;
      }
    }
  }
  __syncthreads();

  // Combine the waves: M = max m_w, sum = sum e^(m_w - M) l_w, acc likewise.
  if (threadIdx.x < D) {
    const int d = threadIdx.x;
    float mw[WAVES], big = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      mw[w] = s_m[w];
      big = fmaxf(big, mw[w]);
    }
    float total = 0.f, sum = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float f = (mw[w] == -INFINITY) ? 0.f : expf(mw[w] - big);
      float part = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) part += s_acc[w][r * LPK + d / 8][d % 8];
      total = fmaf(f, part, total);
      sum = fmaf(f, s_l[w], sum);
    }
    if (splits == 1) {
      out[((size_t)b * query_heads + h) * D + d] = (uint16_t)f32_to_bf16(sum > 0.f ? total / sum : 0.f);
    } else {
      float* rec = partials + (((size_t)b * query_heads + h) * splits + split) * (D + 2);
      rec[2 + d] = total;
      if (d == 0) {
        rec[0] = big;
        rec[1] = sum;
      }
    }
  }
}

// Combine the split records of aoto_decode_attention_*: one block per (b, head),
//   out = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s,  M = max_s m_s; 0 when no key is kept.
// Thread d loads column d of the first kMergeRegSplits records into registers
// before anything waits, so the columns arrive with the (m, l) pairs in one round
// trip; the maximum and the denominator are block reductions of one split per
// thread, the column sums read the weights from LDS. D <= 128 (one column per
// thread) and splits <= kMergeMaxSplits, both checked on the host.
constexpr int kMergeMaxSplits = 1024;
constexpr int kMergeRegSplits = 40;
extern "C" __global__ __launch_bounds__(128) void aoto_decode_attention_merge(const float* __restrict__ partials,
                                                                             int splits, int D,
                                                                             uint16_t* __restrict__ out) {
  __shared__ float s_w[kMergeMaxSplits];
  __shared__ float s_red[4];
  const int bh = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int d = threadIdx.x;
  const bool column = d < D;  // uniform per wave (D is 64 or 128)
  const int dc = column ? d : 0;
  const size_t stride = (size_t)D + 2;
  const float* rec = partials + (size_t)bh * splits * stride;
  float a[kMergeRegSplits];
#pragma unroll
  for (int s = 0; s < kMergeRegSplits; ++s) a[s] = s < splits ? rec[(size_t)s * stride + 2 + dc] : 0.f;
  float m = -INFINITY;
  for (int s = threadIdx.x; s < splits; s += 128) m = fmaxf(m, rec[(size_t)s * stride]);
  m = wave_max(m);
  if (lane == 0) s_red[wave] = m;
  __syncthreads();
  const float M = fmaxf(s_red[0], s_red[1]);
  float den = 0.f;
  for (int s = threadIdx.x; s < splits; s += 128) {
    const float ms = rec[(size_t)s * stride];
    const float ls = rec[(size_t)s * stride + 1];
    const float w = (M == -INFINITY || ms == -INFINITY) ? 0.f : expf(ms - M);
    s_w[s] = w;
    den = fmaf(w, ls, den);
  }
  den = wave_sum(den);
  if (lane == 0) s_red[2 + wave] = den;
  __syncthreads();
  den = s_red[2] + s_red[3];
  float num = 0.f;
#pragma unroll
  for (int s = 0; s < kMergeRegSplits; ++s) {
    const float t = fmaf(s_w[s], a[s], num);
    num = s < splits ? t : num;
  }
  for (int s = kMergeRegSplits; s < splits; ++s) num = fmaf(s_w[s], rec[(size_t)s * stride + 2 + dc], num);
  if (column) out[(size_t)bh * D + d] = (uint16_t)f32_to_bf16(den > 0.f ? num / den : 0.f);
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
// One block of 256 threads; hidden % 8 == 0. The arguments of the loads that
// start the kernel come first, within the 14 preloaded argument dwords
// (cap_hd = cap | head_dim << 22; cap < 2^22, head_dim < 512).
extern "C" __global__ __launch_bounds__(256) void aoto_argmax_finish(
    const unsigned long long* __restrict__ keys, int* __restrict__ step, const uint16_t* __restrict__ cos_table,
    const uint16_t* __restrict__ sin_table, long long* __restrict__ history, int* __restrict__ history_len,
    int count, int cap_hd, uint16_t* __restrict__ rope_rows, long long* __restrict__ token_out,
    const uint16_t* __restrict__ embed, long long embed_rows, int hidden, uint16_t* __restrict__ hidden_out,
    int* __restrict__ error) {
  const int cap = cap_hd & 0x3FFFFF, head_dim = (int)((unsigned)cap_hd >> 22);
  __shared__ unsigned long long s_best[4];
  constexpr int kUnroll = 16;  // keys per thread loaded at once (count <= 4096)
  // Everything that does not depend on the token is read up front, in parallel
  // with the keys: the step state, the history length and the next position's
  // RoPE rows.
  int st[4] = {0, 0, 0, 0};
  if (step != nullptr) {
    st[0] = step[0];
    st[1] = step[1];
    st[2] = step[2];
    st[3] = step[3];
  }
  const int at = history != nullptr ? history_len[0] : 0;
  const int p = st[0] + 1;
  // a position past the tables (the step after the last) keeps the old rows
  const bool rows = rope_rows != nullptr && step != nullptr && p < cap && (int)threadIdx.x < head_dim;
  uint16_t cs = 0, sn = 0;
  if (rows) {
    cs = cos_table[(size_t)p * head_dim + threadIdx.x];
    sn = sin_table[(size_t)p * head_dim + threadIdx.x];
  }
  unsigned long long best = 0;
  if (count <= 256 * kUnroll) {
    unsigned long long v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int i = threadIdx.x + 256 * u;
      v[u] = i < count ? keys[i] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) best = max_u64(best, v[u]);
  } else {
    for (int i = threadIdx.x; i < count; i += 256) best = max_u64(best, keys[i]);
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
  if (rows) {
    rope_rows[threadIdx.x] = cs;
    rope_rows[head_dim + threadIdx.x] = sn;
  }
  __syncthreads();
  const unsigned long long m = max_u64(max_u64(s_best[0], s_best[1]), max_u64(s_best[2], s_best[3]));
  const long long token = argmax_key_index(m);
  if (threadIdx.x == 0) {
    token_out[0] = token;
    if (history != nullptr) {
      history[at] = token;
      history_len[0] = at + 1;
    }
    if (step != nullptr) {
      step[0] = st[0] + 1;
      step[1] = st[1] + 1;
      step[2] = st[2] + 1 == cap ? 0 : st[2] + 1;
      step[3] = st[3] + 1 == cap ? 0 : st[3] + 1;
    }
  }
  if (embed == nullptr) return;
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

// aoto_decode_attention_d{D}_w{WAVES}j{J} and aoto_decode_rope_attention_d{D}_w{WAVES}j{J}.
// The fused ring-step kernel takes the arguments its first loads need in the
// 14 preloaded argument dwords: the row, the RoPE rows, the cache bases, the
// strides (elements, < 2^31) and packed small integers - heads = query_heads |
// kv_heads << 16, starts_qk = query_start | key_start << 16, start_v_width =
// value_start | row_width << 16 (each < 2^16), chunk_cap = chunk | cap << 9
// (chunk < 512, cap < 2^22); the launcher checks the ranges.
#define AOTO_DECODE_ATTENTION_INSTANCE(D, WAVES, J)                                                       \
  extern "C" __global__ __launch_bounds__(64 * WAVES) void aoto_decode_attention_d##D##_w##WAVES##j##J(  \
      const uint16_t* q, uint16_t* kbase, uint16_t* vbase, long long kv_batch_stride,                    \
      long long kv_head_stride, const uint8_t* mask, int mask_batch_stride, int valid, int ring_offset,  \
      int cap, int query_heads, int kv_heads, float scale, int chunk, float* partials, const int* step,  \
      uint16_t* out) {                                                                                   \
    aoto::decode_attention_body<D, WAVES, J, false, false>(                                              \
        q, nullptr, 0, 0, 0, 0, nullptr, nullptr, kbase, vbase, kv_batch_stride, kv_head_stride, mask,  \
        mask_batch_stride, valid, ring_offset, 0, -1, cap, query_heads, kv_heads, scale, chunk, partials, \
        step, nullptr, out);                                                                             \
  }                                                                                                      \
  extern "C" __global__ __launch_bounds__(64 * WAVES) void                                               \
      aoto_decode_rope_attention_d##D##_w##WAVES##j##J(                                                  \
          const uint16_t* row, const uint16_t* rope_rows, uint16_t* kbase, uint16_t* vbase,              \
          int kv_head_stride, int kv_batch_stride, int heads, int starts_qk, int start_v_width,          \
          int chunk_cap, int valid, int ring_offset, int position, int slot, float scale,                \
          float* partials, const int* step, const uint16_t* cos_table, const uint16_t* sin_table,        \
          uint16_t* out) {                                                                               \
    const int query_heads = heads & 0xFFFF, kv_heads = (int)((unsigned)heads >> 16);                     \
    const int query_start = starts_qk & 0xFFFF, key_start = (int)((unsigned)starts_qk >> 16);            \
    const int value_start = start_v_width & 0xFFFF, row_width = (int)((unsigned)start_v_width >> 16);    \
    const int chunk = chunk_cap & 0x1FF, cap = (int)((unsigned)chunk_cap >> 9);                          \
    if (rope_rows != nullptr)                                                                            \
      aoto::decode_attention_body<D, WAVES, J, true, true>(                                              \
          nullptr, row, row_width, query_start, key_start, value_start, cos_table, sin_table, kbase,     \
          vbase, kv_batch_stride, kv_head_stride, nullptr, 0, valid, ring_offset, position, slot, cap,   \
          query_heads, kv_heads, scale, chunk, partials, step, rope_rows, out);                          \
    else                                                                                                 \
      aoto::decode_attention_body<D, WAVES, J, true, false>(                                             \
          nullptr, row, row_width, query_start, key_start, value_start, cos_table, sin_table, kbase,     \
          vbase, kv_batch_stride, kv_head_stride, nullptr, 0, valid, ring_offset, position, slot, cap,   \
          query_heads, kv_heads, scale, chunk, partials, step, nullptr, out);                            \
  }
// Every loads-per-wave count of one head size and block size.
#define AOTO_DECODE_ATTENTION_SHAPES(D, WAVES, J1, J2, J3, J4) \
  AOTO_DECODE_ATTENTION_INSTANCE(D, WAVES, J1)                 \
  AOTO_DECODE_ATTENTION_INSTANCE(D, WAVES, J2)                 \
  AOTO_DECODE_ATTENTION_INSTANCE(D, WAVES, J3)                 \
  AOTO_DECODE_ATTENTION_INSTANCE(D, WAVES, J4)
