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
  const long long tid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
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
// With `step` non-null, valid = step[1] and ring_offset = step[2] (device-side
// step state of a captured decode loop).
//
// Grid (splits, B*Hkv); 256 threads. Each block handles keys
// [split*chunk, min(cap, (split+1)*chunk)) for the G query heads of one kv head:
// LPK lanes per key (D/8 lanes, 16 B each), 64/LPK keys per wave per pass, the
// G scores reduced over the key's lanes with shuffles, the softmax and P.V
// in LDS/registers. With splits == 1 it writes the output; otherwise each block
// stores (max, sum, acc[D]) per head in `partials` and the last block of a kv
// head (an acq_rel counter in `counters`, left at zero afterwards) merges them.
template <int D, int G>
__device__ void decode_attention_body(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kbase,
                                      const uint16_t* __restrict__ vbase, long long kv_batch_stride,
                                      long long kv_head_stride, const uint8_t* __restrict__ mask,
                                      int mask_batch_stride, int valid, int ring_offset, int cap, int kv_heads,
                                      float scale, int chunk, float* __restrict__ partials,
                                      int* __restrict__ counters, const int* __restrict__ step,
                                      uint16_t* __restrict__ out) {
  if (step != nullptr) {
    valid = step[1];
    ring_offset = step[2];
  }
  constexpr int LPK = D / 8;            // lanes per key
  constexpr int KPW = 64 / LPK;         // keys per wave per pass
  constexpr int WAVES = 4;
  constexpr int MAXC = 512;             // keys per block
  __shared__ float s_scores[G][MAXC];
  __shared__ float s_red[G][WAVES];
  __shared__ float s_acc[WAVES][G][D];
  __shared__ int s_last;

  const int split = blockIdx.x;
  const int splits = gridDim.x;
  const int bkv = blockIdx.y;
  const int b = bkv / kv_heads, kvh = bkv % kv_heads;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPK;           // which 8-element slice of the row
  const int kslot = lane / LPK;         // which key of the wave's pass
  const int s0 = split * chunk;
  const int s1 = min(cap, s0 + chunk);
  const int n = max(0, s1 - s0);

  const uint16_t* kh = kbase + (size_t)b * kv_batch_stride + (size_t)kvh * kv_head_stride;
  const uint16_t* vh = vbase + (size_t)b * kv_batch_stride + (size_t)kvh * kv_head_stride;
  const int head0 = kvh * G;
  const int query_heads = kv_heads * G;

  // q slice in registers: G heads x 8 elements, pre-multiplied by nothing
  // (scale applies to the f32 score).
  float qv[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint4 r = reinterpret_cast<const uint4*>(q + ((size_t)b * query_heads + head0 + g) * D)[sub];
    const uint32_t raw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qv[g][2 * i] = bf16_lo(raw[i]);
      qv[g][2 * i + 1] = bf16_hi(raw[i]);
    }
  }

  auto kept = [&](int s) -> bool {
    if (mask != nullptr) return mask[(size_t)b * mask_batch_stride + s] != 0;
    int logical = s - ring_offset;
    logical += logical < 0 ? cap : 0;
    return logical >= cap - valid;
  };

  // Scores.
  float local_max[G];
#pragma unroll
  for (int g = 0; g < G; ++g) local_max[g] = -INFINITY;
  for (int base = wave * KPW; base < n; base += WAVES * KPW) {
    const int i = base + kslot;
    const bool in_range = i < n;
    float part[G];
#pragma unroll
    for (int g = 0; g < G; ++g) part[g] = 0.f;
    if (in_range) {
      const uint4 r = reinterpret_cast<const uint4*>(kh + (size_t)(s0 + i) * D)[sub];
      const uint32_t raw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float k0 = bf16_lo(raw[j]), k1 = bf16_hi(raw[j]);
#pragma unroll
        for (int g = 0; g < G; ++g) part[g] = fmaf(qv[g][2 * j + 1], k1, fmaf(qv[g][2 * j], k0, part[g]));
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) part[g] = group_sum<LPK>(part[g]);
    if (in_range && sub == 0) {
      const bool keep = kept(s0 + i);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float sc = keep ? part[g] * scale : -INFINITY;
        s_scores[g][i] = sc;
        local_max[g] = fmaxf(local_max[g], sc);
      }
    }
  }
  // Block max per head.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = group_max<64>(local_max[g]);
    if (lane == 0) s_red[g][wave] = m;
  }
  __syncthreads();
  float row_max[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = s_red[g][0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) m = fmaxf(m, s_red[g][w]);
    row_max[g] = m;
  }
  __syncthreads();
  // Exponentials and sums.
  float local_sum[G];
#pragma unroll
  for (int g = 0; g < G; ++g) local_sum[g] = 0.f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float sc = s_scores[g][i];
      const float p = (row_max[g] == -INFINITY || sc == -INFINITY) ? 0.f : expf(sc - row_max[g]);
      s_scores[g][i] = p;
      local_sum[g] += p;
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float s = group_sum<64>(local_sum[g]);
    if (lane == 0) s_red[g][wave] = s;
  }
  __syncthreads();
  float row_sum[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) s += s_red[g][w];
    row_sum[g] = s;
  }
  // P.V: each lane accumulates 8 columns of its key slot's rows.
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.f;
  for (int base = wave * KPW; base < n; base += WAVES * KPW) {
    const int i = base + kslot;
    if (i < n) {
      const uint4 r = reinterpret_cast<const uint4*>(vh + (size_t)(s0 + i) * D)[sub];
      const uint32_t raw[4] = {r.x, r.y, r.z, r.w};
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = bf16_lo(raw[j]);
        v[2 * j + 1] = bf16_hi(raw[j]);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = s_scores[g][i];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] = fmaf(p, v[j], acc[g][j]);
      }
    }
  }
  // Reduce over the wave's key slots (lanes with the same `sub`), then waves.
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float a = acc[g][j];
#pragma unroll
      for (int off = LPK; off < 64; off <<= 1) a += __shfl_xor(a, off, 64);
      acc[g][j] = a;
    }
  if (kslot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < 8; ++j) s_acc[wave][g][sub * 8 + j] = acc[g][j];
  }
  __syncthreads();

  if (splits == 1) {
    for (int e = threadIdx.x; e < G * D; e += blockDim.x) {
      const int g = e / D, d = e % D;
      float a = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) a += s_acc[w][g][d];
      const float o = row_sum[g] > 0.f ? a / row_sum[g] : 0.f;
      out[((size_t)b * query_heads + head0 + g) * D + d] = (uint16_t)f32_to_bf16(o);
    }
    return;
  }
  // Partial record per (b, head, split): [max, sum, acc[D]].
  const int rec = D + 2;
  for (int e = threadIdx.x; e < G * D; e += blockDim.x) {
    const int g = e / D, d = e % D;
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) a += s_acc[w][g][d];
    float* p = partials + (((size_t)b * query_heads + head0 + g) * splits + split) * rec;
    p[2 + d] = a;
    if (d == 0) {
      p[0] = row_max[g];
      p[1] = row_sum[g];
    }
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int done = __hip_atomic_fetch_add(counters + bkv, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = done == splits - 1;
    if (s_last) __hip_atomic_store(counters + bkv, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  __atomic_thread_fence(__ATOMIC_ACQUIRE);
  for (int e = threadIdx.x; e < G * D; e += blockDim.x) {
    const int g = e / D, d = e % D;
    const float* p = partials + (((size_t)b * query_heads + head0 + g) * splits) * rec;
    float m = -INFINITY;
    for (int s = 0; s < splits; ++s) m = fmaxf(m, __builtin_nontemporal_load(p + (size_t)s * rec));
    float num = 0.f, den = 0.f;
    if (m != -INFINITY) {
      for (int s = 0; s < splits; ++s) {
        const float ms = __builtin_nontemporal_load(p + (size_t)s * rec);
        if (ms == -INFINITY) continue;
        const float w = expf(ms - m);
        den = fmaf(w, __builtin_nontemporal_load(p + (size_t)s * rec + 1), den);
        num = fmaf(w, __builtin_nontemporal_load(p + (size_t)s * rec + 2 + d), num);
      }
    }
    const float o = den > 0.f ? num / den : 0.f;
    out[((size_t)b * query_heads + head0 + g) * D + d] = (uint16_t)f32_to_bf16(o);
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
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
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

// Order-preserving key of a bf16 value with the index in the low bits so that
// the maximum key is the largest value and, among equal values, the first index.
AOTO_DEVICE unsigned long long argmax_key(uint32_t bits16, int index) {
  uint32_t u = bits16 & 0xFFFFu;
  u = (u & 0x8000u) ? (~u & 0xFFFFu) : (u | 0x8000u);
  if ((bits16 & 0x7FFFu) > 0x7F80u) u = 0;  // NaN never wins
  return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)index);
}

AOTO_DEVICE unsigned long long max_u64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

AOTO_DEVICE unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(v, off, 64);
    v = max_u64(v, o);
  }
  return v;
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
    for (int c = threadIdx.x; c < n / 8; c += blockDim.x) {
      const uint4 r = rv[c];
      const uint32_t raw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        best = max_u64(best, argmax_key(raw[j] & 0xFFFFu, c * 8 + 2 * j));
        best = max_u64(best, argmax_key(raw[j] >> 16, c * 8 + 2 * j + 1));
      }
    }
  } else {
    for (int i = threadIdx.x; i < n; i += blockDim.x) best = max_u64(best, argmax_key(row[i], i));
  }
  best = wave_max_u64(best);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) s_best[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long m = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) m = max_u64(m, s_best[w]);
    const long long token = (long long)(0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFull));
    out[blockIdx.x] = token;
    if (history != nullptr && gridDim.x == 1) {
      const int at = history_len[0];
      history[at] = token;
      history_len[0] = at + 1;
    }
  }
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

#define AOTO_DECODE_ATTENTION_INSTANCE(D, G)                                                              \
  extern "C" __global__ __launch_bounds__(256) void aoto_decode_attention_d##D##_g##G(                   \
      const uint16_t* q, const uint16_t* kbase, const uint16_t* vbase, long long kv_batch_stride,         \
      long long kv_head_stride, const uint8_t* mask, int mask_batch_stride, int valid, int ring_offset,   \
      int cap, int kv_heads, float scale, int chunk, float* partials, int* counters, const int* step,     \
      uint16_t* out) {                                                                                      \
    aoto::decode_attention_body<D, G>(q, kbase, vbase, kv_batch_stride, kv_head_stride, mask,             \
                                      mask_batch_stride, valid, ring_offset, cap, kv_heads, scale, chunk, \
                                      partials, counters, step, out);                                     \
  }
