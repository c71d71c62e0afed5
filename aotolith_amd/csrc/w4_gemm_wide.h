// Long-prefill W4 / W8 GEMM on v_mfma_f32_32x32x16_bf16 with the dequant fused in
// registers and large per-wave tiles.
//
//   Y[m][n] = epilogue( sum_k X[m][k] * bf16(code[n][k] * s[n][k/group]) )
//
// The same product and epilogues as w4_gemm.h (the reference's unpack + tiled
// GEMM, codegen/quantize.py:27-63, codegen/matmul.py:1228-1473, 1721-1742), for
// prompts of hundreds to thousands of rows. What bounds the 16x16x32 kernel there
// is the dequant: every packed word a wave expands to eight bf16 values is used by
// only the wave's own rows, and each wave64 VALU op costs about a third of a
// 16x16x32 product on gfx950. Here a wave owns WM = 128 or 256 rows, so each
// expanded word feeds 4-8 products of 32x32x16 (the faster MFMA shape on gfx950),
// and WN = 32-96 columns, so each X operand read from LDS feeds 2-3 products.
//
// MFMA formulation: C^T = W . X^T per 32x32 tile, so
//   A (32 n x 16 k): lane l holds W[n0 + l%32][k-unit of half l/32]   -> one packed word
//   B (16 k x 32 m): lane l holds X[m0 + l%32][k-unit of half l/32]   -> 16 B of an X row
//   C (32 n x 32 m): lane l, register e holds Y[m0 + l%32][n0 + 8(e/4) + 4(l/32) + e%4]
// A sub-step is 16 k: lane half h supplies one 8-code unit of its row (A) and the
// matching 16 bytes of its X row (B); over a 128-k step lane half h covers units
// 8h .. 8h+7 and sub-step j takes unit 8h + j from both operands, so the sum over
// k is the same, in another order. Each 32 k of a lane half lie in one group
// (group % 32 == 0): two scales per lane and step.
//
// Exact dequant: with n = code + 8 (the nibble's sign bit flipped, 0..15), an
// f16 lane holding 1024 + n (n OR-ed into the mantissa of 1024.0) goes through
// v_fma_mix_f32(1024 + n, s, -1032 s) = code * s exactly (every product and the
// sum are exact in f32: s has 8 significant bits), and one v_cvt_pk_bf16_f32
// rounds two of them to nearest even: bf16(code * s), the reference's unpacked
// value. A nibble 4 bits up gives 1024 + 16 n, taken with s / 16 and -72 s (also
// exact for every bf16 s). Per 8 codes: one shift, four v_bitop3 (mask, sign
// flip and exponent in one op), eight v_fma_mix_f32, four packs.
//
// Block: NW (4 or 8) waves side by side along n. A step is 128 k: its X tile
// [BM][128] and each wave's packed words and scales go from global memory straight
// into LDS (global-to-LDS loads, no VGPRs on the way; X chunks XOR-swizzled so each
// 16-lane phase of an operand read touches 16 bank groups), two or three steps in
// flight, one barrier per step (w4_gemm_wide_body).
#pragma once

#include "common.h"
#include "w4_gemm.h"

namespace aoto {

typedef float wide_f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t wide_u32x4 __attribute__((ext_vector_type(4)));


typedef _Float16 wide_f16x2 __attribute__((ext_vector_type(2)));

// Per-step scale constants of one weight row: {s, s / 16, -1032 s, -72 s} for
// 4-bit codes, {s, -, -1152 s, -} for 8-bit codes (n = code + 128 at 1024 + n).
struct WideScale {
  float s, s16, c0, c1;
};
template <int BITS>
AOTO_DEVICE WideScale wide_scale(float s) {
  if constexpr (BITS == 4) return WideScale{s, s * 0.0625f, s * -1032.0f, s * -72.0f};
  return WideScale{s, 0.f, s * -1152.0f, 0.f};
}

AOTO_DEVICE float mix_lo(uint32_t h, float s, float c) {
  return __builtin_fmaf((float)__builtin_bit_cast(wide_f16x2, h)[0], s, c);
}
AOTO_DEVICE float mix_hi(uint32_t h, float s, float c) {
  return __builtin_fmaf((float)__builtin_bit_cast(wide_f16x2, h)[1], s, c);
}

// (w & m) ^ x in one v_bitop3_b32 (truth table 0x6a over S0, S1, S2; checked
// against the C expression by the GPU tests of every dequantized value). Inside
// the GEMM loop the compiler emits an and and an xor for the C expression, even
// with both constants in registers.
AOTO_DEVICE uint32_t and_xor(uint32_t w, uint32_t m, uint32_t x) {
  uint32_t r;
  asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x6a" : "=v"(r) : "v"(w), "v"(m), "v"(x));
  return r;
}

// The masks and flips of the dequant, held in registers (loop invariants).
struct WideMasks {
  uint32_t m0, m1, x0, x1;
};
template <int BITS>
AOTO_DEVICE WideMasks wide_masks() {
  WideMasks k = BITS == 4 ? WideMasks{0x000F000Fu, 0x00F000F0u, 0x64086408u, 0x64806480u}
                          : WideMasks{0x00FF00FFu, 0x00FF00FFu, 0x64806480u, 0x64806480u};
  asm volatile("" : "+v"(k.m0), "+v"(k.m1), "+v"(k.x0), "+v"(k.x1));
  return k;
}

// bf16(code * s) of the eight 4-bit codes of one word, in k order.
AOTO_DEVICE bf16x8_v wide_dequant(uint32_t w, const WideScale& q, const WideMasks& k) {
  const uint32_t w8 = w >> 8;
  // ((w ^ 0x88888888) & M) | 0x64006400 == (w & M) ^ K: the mask and the exponent bits are disjoint
  const uint32_t h04 = and_xor(w, k.m0, k.x0);   // codes 0, 4: 1024 + n
  const uint32_t h15 = and_xor(w, k.m1, k.x1);   // codes 1, 5: 1024 + 16 n
  const uint32_t h26 = and_xor(w8, k.m0, k.x0);  // codes 2, 6
  const uint32_t h37 = and_xor(w8, k.m1, k.x1);  // codes 3, 7
  const uint32_t p[4] = {cvt_pk_bf16(mix_lo(h04, q.s, q.c0), mix_lo(h15, q.s16, q.c1)),
                         cvt_pk_bf16(mix_lo(h26, q.s, q.c0), mix_lo(h37, q.s16, q.c1)),
                         cvt_pk_bf16(mix_hi(h04, q.s, q.c0), mix_hi(h15, q.s16, q.c1)),
                         cvt_pk_bf16(mix_hi(h26, q.s, q.c0), mix_hi(h37, q.s16, q.c1))};
  return __builtin_bit_cast(bf16x8_v, p);
}

// bf16(code * s) of the eight 8-bit codes of two words (bytes 0..3 of lo, then hi).
AOTO_DEVICE bf16x8_v wide_dequant(uint2 w, const WideScale& q, const WideMasks& k) {
  const uint32_t a02 = and_xor(w.x, k.m0, k.x0), a13 = and_xor(w.x >> 8, k.m0, k.x0);
  const uint32_t b02 = and_xor(w.y, k.m0, k.x0), b13 = and_xor(w.y >> 8, k.m0, k.x0);
  const uint32_t p[4] = {cvt_pk_bf16(mix_lo(a02, q.s, q.c0), mix_lo(a13, q.s, q.c0)),
                         cvt_pk_bf16(mix_hi(a02, q.s, q.c0), mix_hi(a13, q.s, q.c0)),
                         cvt_pk_bf16(mix_lo(b02, q.s, q.c0), mix_lo(b13, q.s, q.c0)),
                         cvt_pk_bf16(mix_hi(b02, q.s, q.c0), mix_hi(b13, q.s, q.c0))};
  return __builtin_bit_cast(bf16x8_v, p);
}

// Scheduling groups (__builtin_amdgcn_sched_group_barrier masks).
constexpr int kSchedVALU = 0x002, kSchedMFMA = 0x008, kSchedVMEMRead = 0x020, kSchedDSRead = 0x100,
              kSchedDSWrite = 0x200;

// One sub-step's interleave: each of its MF products followed by VALU of the
// next sub-step's dequant, one LDS operand read while any remain, and the
// step's X stores / global loads spread over the first products.
template <int MF, int VALU, int DSR, int DSW, int VMEM>
AOTO_DEVICE void wide_interleave() {
  static_for<MF>([&](auto i_c) __attribute__((always_inline)) {
    constexpr int i = decltype(i_c)::value;
    __builtin_amdgcn_sched_group_barrier(kSchedMFMA, 1, 0);
    if constexpr (i < DSR) __builtin_amdgcn_sched_group_barrier(kSchedDSRead, 1, 0);
    if constexpr (i < DSW) __builtin_amdgcn_sched_group_barrier(kSchedDSWrite, 1, 0);
    if constexpr (i < VMEM) __builtin_amdgcn_sched_group_barrier(kSchedVMEMRead, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedVALU, (VALU + MF - 1) / MF, 0);
  });
}

// One 1-KB global -> LDS load of a wave (global_load_lds_dwordx4): lane l's 16
// bytes at `src` land at lds + 16 l. No VGPR holds the data on its way.
AOTO_DEVICE void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
// ... and lane l's 4 bytes at lds + 4 l.
AOTO_DEVICE void dma4(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}
// s_waitcnt with only vmcnt / only lgkmcnt counted (gfx9 encoding).
#define AOTO_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))
#define AOTO_WAIT_LGKMCNT(n) __builtin_amdgcn_s_waitcnt(0xC07F | (((n) & 0xF) << 8))

// Three staging buffers where they fit 160 KB of LDS (X 256 bytes a row, words
// and scales per wave), else two.
constexpr int wide_stages(int bits, int mt, int nt, int np, int nw) {
  return 3 * (32 * mt * 256 + nw * np * nt * (bits / 2) * 1024 + nw * np * nt * 256) <= 160 * 1024 ? 3 : 2;
}

// Split-K: blockIdx.z takes the reduction slice [z*kslice, min(K, (z+1)*kslice));
// with `partials` non-null the block stores f32 tiles to partials[z][m][n] (gate
// at [z], up at [splits + z] for PAIRED), the layout aoto_w4_gemm_reduce* read.
//
// Staging: a step is 128 k. Its X tile [BM rows][128 k] (256 bytes a row) goes
// straight from global memory into LDS with 1-KB loads (four rows each), chunk c
// of row r at slot c ^ (r & 15), so the 16 lanes of each operand-read phase (16
// rows, one chunk) hit 16 different bank groups. Each wave's words (lane l: the
// 8 units 8h .. 8h+7 of its row, h = l / 32) and scale dword land in the wave's own
// LDS slots the same way. STAGES buffers of each: the loads of step st + STAGES - 1
// are issued after the barrier of step st - 1 (into the buffers step st - 1 has
// finished with) and waited for just before the barrier of step st + STAGES - 2.
template <int BITS, int WM, int WN, int NW, bool BIAS, bool RESIDUAL, bool GATE, bool PAIRED, int STAGES>
__device__ void w4_gemm_wide_body(const uint16_t* __restrict__ X, const typename GemmWord<BITS>::type* __restrict__ words,
                                  const uint16_t* __restrict__ scales, const uint16_t* __restrict__ bias,
                                  const uint16_t* __restrict__ residual, const uint16_t* __restrict__ gate,
                                  uint16_t* __restrict__ Y, int M, int N, int K, int group, int kslice,
                                  float* __restrict__ partials,
                                  const typename GemmWord<BITS>::type* __restrict__ up_words,
                                  const uint16_t* __restrict__ up_scales) {
  static_assert(!(PAIRED && (BIAS || RESIDUAL || GATE)), "the paired form has its own epilogue");
  static_assert(WM % 32 == 0 && WN % 32 == 0 && (NW == 4 || NW == 8), "tile shape");
  constexpr int MT = WM / 32, NT = WN / 32, NP = PAIRED ? 2 : 1;
  constexpr int BM = WM, BN = WN * NW;
  constexpr int BK = 128;
  constexpr int XROW = BK * 2;                 // bytes of a staged X row
  constexpr int XDW = BM * XROW / 1024 / NW;   // 1-KB X loads per wave and step
  static_assert(BM * XROW % (1024 * NW) == 0, "whole X loads per wave");
  constexpr int WV = BITS / 4;                 // 16-byte vectors per lane and 4 units
  constexpr int WD = 2 * WV;                   // 1-KB word loads per (matrix, n tile) and step
  constexpr int WSLOT = NP * NT * WD * 1024;   // bytes of a wave's words per step
  constexpr int SSLOT = NP * NT * 256;         // bytes of a wave's scale dwords per step
  static_assert(STAGES == 2 || STAGES == 3, "two or three staging buffers");
  static_assert(STAGES * (BM * XROW + NW * WSLOT + NW * SSLOT) <= 160 * 1024, "staging fits the CU's LDS");
  // One LDS object per buffer, so the compiler's wait analysis keeps the loads
  // into one buffer apart from the reads of another.
  constexpr int S3 = STAGES == 3 ? 1 : 0;
  __shared__ __attribute__((aligned(16))) uint8_t xs0[BM * XROW];
  __shared__ __attribute__((aligned(16))) uint8_t xs1[BM * XROW];
  __shared__ __attribute__((aligned(16))) uint8_t xs2[S3 ? BM * XROW : 16];
  __shared__ __attribute__((aligned(16))) uint8_t ws0[NW * WSLOT];
  __shared__ __attribute__((aligned(16))) uint8_t ws1[NW * WSLOT];
  __shared__ __attribute__((aligned(16))) uint8_t ws2[S3 ? NW * WSLOT : 16];
  __shared__ __attribute__((aligned(16))) uint8_t ss0[NW * SSLOT];
  __shared__ __attribute__((aligned(16))) uint8_t ss1[NW * SSLOT];
  __shared__ __attribute__((aligned(16))) uint8_t ss2[S3 ? NW * SSLOT : 16];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform, for LDS load targets
  const int col = lane & 31, half = lane >> 5;
  const int n_wave = blockIdx.x * BN + wave * WN;
  const int m_block = blockIdx.y * BM;
  constexpr int m_wave = 0;  // every wave covers the block's rows
  const int kw = K >> 3;                      // 8-code units per weight row
  const int groups = K / group;
  const int gshift = __builtin_ctz(group);    // group: a power of two >= 32
  const int kb = blockIdx.z * kslice;
  const int steps = (min(K, kb + kslice) - kb) / BK;

  wide_f32x16 acc[NP][NT][MT];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int u = 0; u < MT; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[p][t][u][e] = 0.f;

  // This lane's weight rows (clamped: rows past N compute values never stored),
  // as bytes, and its X load sources (rows past M clamped the same way).
  const uint8_t* wsrc[NP][NT];
  const uint8_t* ssrc[NP][NT];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int row = min(n_wave + 32 * t + col, N - 1);
      wsrc[p][t] = reinterpret_cast<const uint8_t*>((p == 0 ? words : up_words) + (size_t)row * kw) +
                   half * 8 * 4 * WV;  // units 8h ..: 4 * WV bytes per unit
      ssrc[p][t] = reinterpret_cast<const uint8_t*>((p == 0 ? scales : up_scales) + (size_t)row * groups);
    }
  const uint8_t* xsrc[XDW];
#pragma unroll
  for (int i = 0; i < XDW; ++i) {
    const int r = 4 * (wave * XDW + i) + (lane >> 4);
    const int c = (lane & 15) ^ (r & 15);
    xsrc[i] = reinterpret_cast<const uint8_t*>(X + (size_t)min(m_block + r, M - 1) * K + 8 * c);
  }
  // The B operand read of sub-step j, m tile u: row m_wave + 32u + col, chunk
  // (8h + j) ^ (col & 15), i.e. xrd ^ (16 j) + 8192 u.
  const int xrd = (m_wave + col) * XROW + (((8 * half) ^ (col & 15)) << 4);

  // the loads of step st into buffer set (xb, wb, sb); steps past the slice re-read the last
  auto issue = [&](int st, uint8_t* xb, uint8_t* wb, uint8_t* sb) __attribute__((always_inline)) {
    const int k0 = kb + min(st, steps - 1) * BK;
#pragma unroll
    for (int i = 0; i < XDW; ++i) dma16(xsrc[i] + 2 * k0, xb + (wave_u * XDW + i) * 1024);
    const int wbyte = (k0 >> 3) * 4 * WV;
    // scale dword: group 32 -> the two groups of the half's 64 k; larger -> the
    // aligned pair holding the half's group (rows hold an even number of groups)
    const int sidx = (k0 + 64 * half) >> gshift;
    const int sbyte = (sidx & ~1) * 2;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int d = 0; d < WD; ++d)
          dma16(wsrc[p][t] + wbyte + 16 * d, wb + wave_u * WSLOT + ((p * NT + t) * WD + d) * 1024);
        dma4(ssrc[p][t] + sbyte, sb + wave_u * SSLOT + (p * NT + t) * 256);
      }
  };

  wide_u32x4 wlo[NP][NT][WV], whi[NP][NT][WV];  // a lane's units 8h .. 8h+3 and 8h+4 .. 8h+7
  float flo[NP][NT], fhi[NP][NT];                // the scales of those units (constants per sub-step:
                                                 // precomputed for the step, they let the compiler
                                                 // hoist every sub-step's dequant: 446 against 276 VGPRs)
  const WideMasks km = wide_masks<BITS>();
  bf16x8_v a[2][NP][NT];                         // dequantized operands: current / next sub-step
  bf16x8_v b[2][MT];                             // X operands: current / next sub-step
  auto read_w = [&](auto hi_c, const uint8_t* wb) __attribute__((always_inline)) {
    constexpr int hi = decltype(hi_c)::value;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int e = 0; e < WV; ++e) {
          const wide_u32x4 v = *reinterpret_cast<const wide_u32x4*>(
              wb + wave_u * WSLOT + ((p * NT + t) * WD + hi * WV + e) * 1024 + 16 * lane);
          if constexpr (hi) whi[p][t][e] = v; else wlo[p][t][e] = v;
        }
  };
  // Scale constants of step st: units 8h .. 8h+3 and 8h+4 .. 8h+7 lie in one group
  // each (group >= 32); a step past the slice (odd step counts in the unrolled
  // loop) takes scale 0, so its products add exactly zero.
  auto read_s = [&](const uint8_t* sb, int st) __attribute__((always_inline)) {
    const int k0 = kb + min(st, steps - 1) * BK;
    const int slo = ((k0 + 64 * half) >> gshift) & 1, shi = ((k0 + 64 * half + 32) >> gshift) & 1;
    const bool live = st < steps;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t sw = *reinterpret_cast<const uint32_t*>(sb + wave_u * SSLOT + (p * NT + t) * 256 + 4 * lane);
        flo[p][t] = live ? bf16_to_f32((sw >> (16 * slo)) & 0xFFFFu) : 0.f;
        fhi[p][t] = live ? bf16_to_f32((sw >> (16 * shi)) & 0xFFFFu) : 0.f;
      }
  };
  auto read_b = [&](auto into_c, const uint8_t* xb, int j) __attribute__((always_inline)) {
    constexpr int into = decltype(into_c)::value;
    const uint8_t* base = xb + (xrd ^ (16 * j));
#pragma unroll
    for (int u = 0; u < MT; ++u) b[into][u] = *reinterpret_cast<const bf16x8_v*>(base + 32 * XROW * u);
  };
  // Operands of sub-step j of the current step.
  auto dequant = [&](auto into_c, auto j_c) __attribute__((always_inline)) {
    constexpr int into = decltype(into_c)::value, j = decltype(j_c)::value;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const WideScale q = wide_scale<BITS>(j < 4 ? flo[p][t] : fhi[p][t]);
        const wide_u32x4(&wv)[WV] = j < 4 ? wlo[p][t] : whi[p][t];
        constexpr int jj = j & 3;
        if constexpr (BITS == 4) {
          a[into][p][t] = wide_dequant(wv[0][jj], q, km);
        } else {
          const wide_u32x4& h = wv[jj >> 1];
          a[into][p][t] = wide_dequant(make_uint2(h[(jj & 1) * 2], h[(jj & 1) * 2 + 1]), q, km);
        }
      }
  };
  auto products = [&](auto from_c) __attribute__((always_inline)) {
    constexpr int from = decltype(from_c)::value;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int u = 0; u < MT; ++u)
          acc[p][t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[from][p][t], b[from][u], acc[p][t][u], 0, 0, 0);
  };
  constexpr int MF = NP * NT * MT;                     // products per sub-step
  constexpr int DQ = NP * NT * (BITS == 4 ? 17 : 18);  // dequant VALU per sub-step

  constexpr int DPS = XDW + NP * NT * (WD + 1);  // a wave's loads per step
  // Prologue: step 0 staged, steps 1 .. STAGES - 1 in flight, sub-step 0's operands ready.
  issue(0, xs0, ws0, ss0);
  issue(1, xs1, ws1, ss1);
  if constexpr (S3) {
    issue(2, xs2, ws2, ss2);
    AOTO_WAIT_VMCNT(2 * DPS);
  } else {
    AOTO_WAIT_VMCNT(DPS);
  }
  __builtin_amdgcn_s_barrier();
  read_w(std::integral_constant<int, 0>{}, ws0);
  read_s(ss0, 0);
  read_b(std::integral_constant<int, 0>{}, xs0, 0);
  dequant(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});

  // Step st: sub-step j's products run while sub-step j + 1's operands are read
  // and dequantized. Before sub-step 7: wait for step st + 1's loads and this
  // step's reads, barrier; then step st + 2's loads go into this step's buffers
  // and sub-step 7 overlaps step st + 1's first reads and dequant.
  auto step = [&](int st, uint8_t* xc, uint8_t* wc, uint8_t* sc, uint8_t* xn, uint8_t* wn, uint8_t* sn)
                  __attribute__((always_inline)) {
    static_for<7>([&](auto j_c) __attribute__((always_inline)) {
      constexpr int j = decltype(j_c)::value;
      using Cur = std::integral_constant<int, j & 1>;
      using Nxt = std::integral_constant<int, 1 - (j & 1)>;
      read_b(Nxt{}, xc, j + 1);
      if constexpr (j == 0) read_w(std::integral_constant<int, 1>{}, wc);
      dequant(Nxt{}, std::integral_constant<int, j + 1>{});
      products(Cur{});
      wide_interleave<MF, DQ, MT + (j == 0 ? NP * NT * WV : 0), 0, 0>();
      __builtin_amdgcn_sched_barrier(0);  // keep each sub-step's work in its sub-step
    });
    AOTO_WAIT_VMCNT((STAGES - 2) * DPS);  // step st + 1's loads are in
    AOTO_WAIT_LGKMCNT(0);
    __builtin_amdgcn_s_barrier();
    issue(st + STAGES, xc, wc, sc);
    read_w(std::integral_constant<int, 0>{}, wn);
    read_s(sn, st + 1);
    read_b(std::integral_constant<int, 0>{}, xn, 0);
    dequant(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    products(std::integral_constant<int, 1>{});
    constexpr int XL = XDW + NP * NT * (WD + 1);
    wide_interleave<MF, DQ + 8, MT + NP * NT * (WV + 1), 0, XL>();
    __builtin_amdgcn_sched_barrier(0);
  };
  if constexpr (S3) {
    for (int st = 0; st < steps; st += 3) {
      step(st, xs0, ws0, ss0, xs1, ws1, ss1);
      step(st + 1, xs1, ws1, ss1, xs2, ws2, ss2);
      step(st + 2, xs2, ws2, ss2, xs0, ws0, ss0);
    }
  } else {
    for (int st = 0; st < steps; st += 2) {
      step(st, xs0, ws0, ss0, xs1, ws1, ss1);
      step(st + 1, xs1, ws1, ss1, xs0, ws0, ss0);
    }
  }
  // The last rounds' loads (of steps past the slice) still land in LDS: wait for
  // them before the block ends (split-K) or reuses the buffers (epilogue).
  AOTO_WAIT_VMCNT(0);

  if (partials != nullptr) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float* part = partials + ((size_t)p * gridDim.z + blockIdx.z) * M * N;
#pragma unroll
      for (int u = 0; u < MT; ++u) {
        const int m = m_block + m_wave + 32 * u + col;
        if (m >= M) continue;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int n = n_wave + 32 * t + 8 * g + 4 * half;
            if (n >= N) continue;
            *reinterpret_cast<float4*>(part + (size_t)m * N + n) =
                make_float4(acc[p][t][u][4 * g], acc[p][t][u][4 * g + 1], acc[p][t][u][4 * g + 2],
                            acc[p][t][u][4 * g + 3]);
          }
      }
    }
    return;
  }
  // Epilogue (w4_gemm.h's rounding points). The lane's accumulators hold
  // Y[m][n .. n+4) for one row per lane and register quad, so direct stores would
  // write 16 bytes into each of 32 rows per instruction. Each 32 x 32 sub-tile
  // instead goes through the wave's own 4.5-KB LDS slot (f32 rows 144 bytes apart:
  // the 16 lanes of a write phase hit 16 bank groups) and comes back eight lanes
  // per row: 64 contiguous bytes of residual, gate and output per row.
  // Staging after the loop reuses the X buffers, once every wave is past them.
  __syncthreads();
  float* slot = reinterpret_cast<float*>((wave < 4 ? xs0 : xs1) + (wave & 3) * 4608);
  static_assert(BM * XROW >= 4 * 4608, "four epilogue slots per X buffer");
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n0 = n_wave + 32 * t;
    float4 bcol = make_float4(0.f, 0.f, 0.f, 0.f);  // bias of this lane's read-back columns
    if constexpr (BIAS) {
      const uint2 bb = *reinterpret_cast<const uint2*>(bias + min(n0 + 4 * (lane & 7), N - 4));
      bcol = make_float4(bf16_lo(bb.x), bf16_hi(bb.x), bf16_lo(bb.y), bf16_hi(bb.y));
    }
#pragma unroll
    for (int u = 0; u < MT; ++u) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float v[4] = {acc[0][t][u][4 * g], acc[0][t][u][4 * g + 1], acc[0][t][u][4 * g + 2], acc[0][t][u][4 * g + 3]};
        if constexpr (PAIRED) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float gt = round_bf16(v[i]);
            v[i] = acc[NP - 1][t][u][4 * g + i] * (gt / (1.0f + expf(-gt)));
          }
        }
        *reinterpret_cast<float4*>(slot + col * 36 + 8 * g + 4 * half) = make_float4(v[0], v[1], v[2], v[3]);
      }
      // read back: lane l takes row l / 8 + 8 q, columns 4 (l % 8) .. + 4
      const int n = n0 + 4 * (lane & 7);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = (lane >> 3) + 8 * q;
        const int m = m_block + m_wave + 32 * u + r;
        const float4 f = *reinterpret_cast<const float4*>(slot + r * 36 + 4 * (lane & 7));
        if (m >= M || n >= N) continue;
        float v[4] = {f.x, f.y, f.z, f.w};
        if constexpr (BIAS) {
          v[0] += bcol.x;
          v[1] += bcol.y;
          v[2] += bcol.z;
          v[3] += bcol.w;
        }
        if constexpr (RESIDUAL) {
          const uint2 rr = *reinterpret_cast<const uint2*>(residual + (size_t)m * N + n);
          v[0] += bf16_lo(rr.x);
          v[1] += bf16_hi(rr.x);
          v[2] += bf16_lo(rr.y);
          v[3] += bf16_hi(rr.y);
        }
        if constexpr (GATE) {
          const uint2 gg = *reinterpret_cast<const uint2*>(gate + (size_t)m * N + n);
          const float gv[4] = {bf16_lo(gg.x), bf16_hi(gg.x), bf16_lo(gg.y), bf16_hi(gg.y)};
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = v[i] * (gv[i] / (1.0f + expf(-gv[i])));
        }
        *reinterpret_cast<uint2*>(Y + (size_t)m * N + n) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
    }
  }
}

}  // namespace aoto

// aoto_w{BITS}_gemm_w{MT}x{NT}x{NW}_b{BIAS}_r{RES}_g{GATE}: WM = 32 MT rows and
// WN = 32 NT columns per wave, NW waves along n.
#define AOTO_GEMM_WIDE_INSTANCE(BITS, MT, NT, NW, BIAS, RES, GATE)                                         \
  extern "C" __global__ __launch_bounds__(64 * NW, 1) void                                                  \
      aoto_w##BITS##_gemm_w##MT##x##NT##x##NW##_b##BIAS##_r##RES##_g##GATE(                                 \
          const uint16_t* X, const aoto::GemmWord<BITS>::type* words, const uint16_t* scales,               \
          const uint16_t* bias, const uint16_t* residual, const uint16_t* gate, uint16_t* Y, int M, int N,  \
          int K, int group, int kslice, float* partials) {                                                  \
    aoto::w4_gemm_wide_body<BITS, 32 * MT, 32 * NT, NW, BIAS, RES, GATE, false,                            \
                            aoto::wide_stages(BITS, MT, NT, 1, NW)>(                                        \
        X, words, scales, bias, residual, gate, Y, M, N, K, group, kslice, partials, nullptr, nullptr);     \
  }
#define AOTO_GEMM_WIDE_EPILOGUES(BITS, MT, NT, NW)   \
  AOTO_GEMM_WIDE_INSTANCE(BITS, MT, NT, NW, 0, 0, 0) \
  AOTO_GEMM_WIDE_INSTANCE(BITS, MT, NT, NW, 1, 0, 0) \
  AOTO_GEMM_WIDE_INSTANCE(BITS, MT, NT, NW, 0, 1, 0) \
  AOTO_GEMM_WIDE_INSTANCE(BITS, MT, NT, NW, 0, 0, 1)
// aoto_w{BITS}_gemm_w{MT}x{NT}x{NW}_paired: the MLP's gate/up pair in one pass.
#define AOTO_GEMM_WIDE_PAIRED_INSTANCE(BITS, MT, NT, NW)                                                   \
  extern "C" __global__ __launch_bounds__(64 * NW, 1) void aoto_w##BITS##_gemm_w##MT##x##NT##x##NW##_paired( \
      const uint16_t* X, const aoto::GemmWord<BITS>::type* words, const uint16_t* scales,                  \
      const aoto::GemmWord<BITS>::type* up_words, const uint16_t* up_scales, uint16_t* Y, int M, int N,    \
      int K, int group, int kslice, float* partials) {                                                     \
    aoto::w4_gemm_wide_body<BITS, 32 * MT, 32 * NT, NW, false, false, false, true,                         \
                            aoto::wide_stages(BITS, MT, NT, 2, NW)>(                                        \
        X, words, scales, nullptr, nullptr, nullptr, Y, M, N, K, group, kslice, partials, up_words,        \
        up_scales);                                                                                        \
  }
