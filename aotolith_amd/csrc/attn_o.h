// Ring decode step of one layer's attention fused with its o projection:
//
//   attn  = GQA attention of the step's query (RoPE applied) over the layer's
//           ring cache, the new key/value standing in at `slot`;
//   hidden[n] = bf16(hidden[n] + sum_k Wo[n][k] * attn[k])   (W4 GEMV + residual)
//
// The two nodes of the reference's decode graph (decode attention,
// codegen/attention.py:447-656, then the packed o-projection GEMV with its
// residual epilogue, codegen/matmul.py:542-739) become one launch. The o GEMV
// needs every head's output, and blocks of one launch cannot exchange data
// without a grid-wide fence (measured at several microseconds on MI355X), so
// every block recomputes the whole attention for itself: for small windows
// (D = 64, one or two kv heads, <= 64 keys per wave) that is a few thousand
// FMAs per lane over K/V rows that sit in L2, cheaper than the kernel boundary
// and the o GEMV's own load round trips it removes. Each block then runs its
// 16 rows of the o GEMV from LDS.
//
// Block: 512 threads, 8 waves. Wave w works on kv head g = w / WPK and keys
// kb*64 + lane (kb = w % WPK, WPK = 8 / kv_heads). Rounding points are those of
// the two separate kernels: q and k rotated and rounded to bf16, scores and
// softmax in f32 (exact bf16 products), P.V in f32, the attention output
// rounded to bf16, then the o GEMV of aoto_w4_gemv (bf16 nibble pairs against
// x pairs, f32 accumulation, one rounding after the residual add).
#pragma once

#include "common.h"
#include "w4_gemv.h"
#include "w4_gemv_stream.h"

namespace aoto {

constexpr int kAttnOThreads = 512;
constexpr int kAttnORows = 16;  // o-projection rows per block (32 lanes each)

struct AttnOArgs {
  const uint16_t* row;        // q/k/v projection row [(Hq + 2 Hkv) * 64] bf16
  const uint16_t* cos_table;  // [cap][64] (used when rope_rows is null)
  const uint16_t* sin_table;
  const uint16_t* rope_rows;  // [2][64]: cos and sin rows of the step's position, or null
  uint16_t* keys;             // layer's key window [Hkv][cap][64]
  uint16_t* values;           // layer's value window [Hkv][cap][64]
  const int* step;            // {position, valid, ring_offset, slot}
  const uint4* words;         // o projection [N][Hq*64/32] 16-byte chunks
  const uint16_t* scales;     // [N][Hq*64/64] bf16
  uint16_t* hidden;           // [N] residual in, output out
  int query_heads, kv_heads, cap, n_out;
  float scale;
};

extern "C" __global__ __launch_bounds__(kAttnOThreads) void aoto_decode_attention_o_d64(AttnOArgs a) {
  constexpr int D = 64;
  __shared__ __attribute__((aligned(16))) uint32_t s_q[16][D / 2];   // rotated queries, bf16 pairs
  __shared__ __attribute__((aligned(16))) uint16_t s_knew[2][D];
  __shared__ __attribute__((aligned(16))) uint16_t s_vnew[2][D];
  __shared__ __attribute__((aligned(16))) uint4 s_v[8][64][D / 8];   // each wave's value rows
  __shared__ __attribute__((aligned(16))) float s_p[8][8][64];       // probabilities [wave][head][key]
  __shared__ __attribute__((aligned(16))) float s_o[8][8][D];        // partial outputs [wave][head][dim]
  __shared__ float s_max[8][8], s_sum[8][8];
  __shared__ __attribute__((aligned(16))) uint4 s_x[D * 16 / 8];     // attention output, GEMV pair layout
  __shared__ float s_csum[D * 16 / 32];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hq = a.query_heads, hkv = a.kv_heads, group = hq / hkv;
  const int wpk = 8 / hkv;
  const int g = wave / wpk, kb = wave % wpk;
  const int K = hq * D;            // o projection reduction
  const int nch = K >> 5;          // 32-code chunks per o row
  const int width = (hq + 2 * hkv) * D;

  // -- loads that depend on nothing: this block's o rows, the K/V rows, the q/k/v row
  const int orow_local = (threadIdx.x >> 5);           // 0..15
  const int ochunk = threadIdx.x & 31;
  const int orow = min(blockIdx.x * kAttnORows + orow_local, a.n_out - 1);
  const int oc = min(ochunk, nch - 1);
  const uint4 ow = a.words[(size_t)orow * nch + oc];
  const uint32_t osc = reinterpret_cast<const uint32_t*>(a.scales)[(size_t)orow * (nch >> 2) + (oc >> 2)];
  const uint32_t ores = a.hidden[orow];

  const int key = kb * 64 + lane;
  const int kc = min(key, a.cap - 1);
  const uint4* krow = reinterpret_cast<const uint4*>(a.keys + ((size_t)g * a.cap + kc) * D);
  const uint4* vrow = reinterpret_cast<const uint4*>(a.values + ((size_t)g * a.cap + kc) * D);
  uint4 kv[8], vv[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) kv[c] = krow[c];
#pragma unroll
  for (int c = 0; c < 8; ++c) vv[c] = vrow[c];

  const int position = a.step[0], valid = a.step[1], ring_offset = a.step[2], slot = a.step[3];

  // -- RoPE of q and the new k (f32, one rounding), new v copied; into LDS.
  // Pair p of the q/k/v row holds elements 2p, 2p+1; the RoPE partner is D/2 away.
  const uint32_t* rw = reinterpret_cast<const uint32_t*>(a.row);
  const int pairs = width >> 1;
  for (int p = threadIdx.x; p < pairs; p += kAttnOThreads) {
    const int e0 = 2 * p;
    const int dd = e0 & (D - 1);
    const uint32_t rx = rw[p];
    const uint32_t rp = rw[(dd < D / 2 ? e0 + D / 2 : e0 - D / 2) >> 1];
    const uint16_t* crow = a.rope_rows != nullptr ? a.rope_rows : a.cos_table + (size_t)position * D;
    const uint16_t* srow = a.rope_rows != nullptr ? a.rope_rows + D : a.sin_table + (size_t)position * D;
    const uint32_t cs = reinterpret_cast<const uint32_t*>(crow)[dd >> 1];
    const uint32_t sn = reinterpret_cast<const uint32_t*>(srow)[dd >> 1];
    const int region = e0 < hq * D ? 0 : (e0 < (hq + hkv) * D ? 1 : 2);
    const float sign = dd < D / 2 ? -1.f : 1.f;
    const float r0 = bf16_lo(rx) * bf16_lo(cs) + sign * bf16_lo(rp) * bf16_lo(sn);
    const float r1 = bf16_hi(rx) * bf16_hi(cs) + sign * bf16_hi(rp) * bf16_hi(sn);
    if (region == 0) {
      s_q[e0 / D][dd >> 1] = pack_bf16x2(r0, r1);
    } else if (region == 1) {
      reinterpret_cast<uint32_t*>(s_knew[(e0 - hq * D) / D])[dd >> 1] = pack_bf16x2(r0, r1);
    } else {
      reinterpret_cast<uint32_t*>(s_vnew[(e0 - (hq + hkv) * D) / D])[dd >> 1] = rx;
    }
  }
  __syncthreads();

  // -- scores: this lane's key against the group's queries (one lane per key)
  // The new key/value stand in at `slot` (selects, not a branch: a divergent
  // whole-array assignment sends the arrays to scratch).
  const bool at_slot = key < a.cap && kc == slot;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint4 kn = reinterpret_cast<const uint4*>(s_knew[g])[c];
    const uint4 vn = reinterpret_cast<const uint4*>(s_vnew[g])[c];
    kv[c] = make_uint4(at_slot ? kn.x : kv[c].x, at_slot ? kn.y : kv[c].y, at_slot ? kn.z : kv[c].z,
                       at_slot ? kn.w : kv[c].w);
    vv[c] = make_uint4(at_slot ? vn.x : vv[c].x, at_slot ? vn.y : vv[c].y, at_slot ? vn.z : vv[c].z,
                       at_slot ? vn.w : vv[c].w);
  }
  int logical = kc - ring_offset;
  logical += logical < 0 ? a.cap : 0;
  const bool kept = key < a.cap && logical >= a.cap - valid;
#pragma unroll
  for (int c = 0; c < 8; ++c) s_v[wave][lane][c] = vv[c];
  float sc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float dot = 0.f;
    if (i < group) {
      const uint4* qv = reinterpret_cast<const uint4*>(s_q[g * group + i]);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint4 q4 = qv[c];
        dot = dot2_bf16(kv[c].x, q4.x, dot);
        dot = dot2_bf16(kv[c].y, q4.y, dot);
        dot = dot2_bf16(kv[c].z, q4.z, dot);
        dot = dot2_bf16(kv[c].w, q4.w, dot);
      }
    }
    sc[i] = kept ? dot * a.scale : -INFINITY;
    const float m = wave_max(sc[i]);
    if (lane == 0) s_max[wave][i] = m;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float m = s_max[g * wpk][i];
    for (int w = 1; w < wpk; ++w) m = fmaxf(m, s_max[g * wpk + w][i]);
    const float p = (sc[i] == -INFINITY) ? 0.f : expf(sc[i] - m);
    s_p[wave][i][lane] = p;
    const float t = wave_sum(p);
    if (lane == 0) s_sum[wave][i] = t;
  }
  __syncthreads();

  // -- P.V over this wave's 64 keys: lane (head i = lane / 8, dims 8*(lane % 8) ..)
  {
    const int i = lane >> 3, dg = lane & 7;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const float4* pr = reinterpret_cast<const float4*>(s_p[wave][i]);
#pragma unroll 4
    for (int s4 = 0; s4 < 16; ++s4) {
      const float4 p4 = pr[s4];
      const float pp[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint4 v = s_v[wave][s4 * 4 + e][dg];
        acc[0] = fmaf(pp[e], bf16_lo(v.x), acc[0]);
        acc[1] = fmaf(pp[e], bf16_hi(v.x), acc[1]);
        acc[2] = fmaf(pp[e], bf16_lo(v.y), acc[2]);
        acc[3] = fmaf(pp[e], bf16_hi(v.y), acc[3]);
        acc[4] = fmaf(pp[e], bf16_lo(v.z), acc[4]);
        acc[5] = fmaf(pp[e], bf16_hi(v.z), acc[5]);
        acc[6] = fmaf(pp[e], bf16_lo(v.w), acc[6]);
        acc[7] = fmaf(pp[e], bf16_hi(v.w), acc[7]);
      }
    }
    float4* o = reinterpret_cast<float4*>(&s_o[wave][i][dg * 8]);
    o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  __syncthreads();

  // -- combine the waves of each kv group: attention output (bf16) in GEMV pair layout
  // thread t < K/8 builds word t: elements 8t .. 8t+7 of head h = 8t / 64.
  if ((int)threadIdx.x < (K >> 3)) {
    const int t = threadIdx.x;
    const int h = (8 * t) / D, d0 = (8 * t) & (D - 1);
    const int gg = h / group, i = h % group;
    float l = 0.f;
    for (int w = 0; w < wpk; ++w) l += s_sum[gg * wpk + w][i];
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = 0.f;
      for (int w = 0; w < wpk; ++w) acc += s_o[gg * wpk + w][i][d0 + e];
      v[e] = round_bf16(l > 0.f ? acc / l : 0.f);
    }
    uint4 out;
    out.x = pack_bf16x2(v[0], v[4]);
    out.y = pack_bf16x2(v[1], v[5]);
    out.z = pack_bf16x2(v[2], v[6]);
    out.w = pack_bf16x2(v[3], v[7]);
    s_x[t] = out;
    float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    if ((t & 3) == 0) s_csum[t >> 2] = sum;
  }
  // block 0 commits the step's (k_rot, v) to the ring at `slot`
  if (blockIdx.x == 0 && (int)threadIdx.x < hkv * D) {
    const int h = threadIdx.x / D, d = threadIdx.x % D;
    a.keys[((size_t)h * a.cap + slot) * D + d] = s_knew[h][d];
    a.values[((size_t)h * a.cap + slot) * D + d] = s_vnew[h][d];
  }
  __syncthreads();

  // -- o projection: 32 lanes per row, one 32-code chunk each, residual epilogue
  const bool valid_chunk = ochunk < nch;
  const float s = ((oc >> 1) & 1) ? bf16_hi(osc) : bf16_lo(osc);
  float total = (chunk_dot_fast(ow, s_x + oc * 4) - 136.f * s_csum[oc]) * (valid_chunk ? s : 0.f);
  total = group_sum<32>(total);
  const int out_row = blockIdx.x * kAttnORows + orow_local;
  if (ochunk == 0 && out_row < a.n_out) a.hidden[out_row] = (uint16_t)f32_to_bf16(bf16_to_f32(ores) + total);
}

}  // namespace aoto
