// Prefill W4 GEMM with each packed tile dequantized once per block into LDS (long
// prompts on 256-row blocks of 8 waves; short prompts on 128-row blocks of 4 waves:
// the paired gate/up, and single projections as split-K partials).
//
//   Y[m][n] = epilogue( sum_k X[m][k] * bf16(code[n][k] * s[n][k/group]) )
//
// The product, rounding points and epilogues of w4_gemm_wide.h (the reference's
// unpack + tiled GEMM, codegen/quantize.py:27-63, codegen/matmul.py:1228-1473,
// 1721-1742). There each wave expands the packed words of its own columns in its
// registers, so a word feeds the products of that wave's 128 rows only; on gfx950
// the expansion's VALU ops take issue cycles from the matrix products (a copy of
// that kernel with the expansion removed runs 18-20% faster at 2048 rows, one that
// keeps the expansion but feeds raw words to the products runs no faster than the
// original: the cost is the VALU count, not the dependency). Here a block of 8
// waves (two per SIMD) takes BM = 256 rows of X and 128 weight rows (128 columns,
// or 64 gate + 64 up columns of the paired form) or 192 (192 columns). Each 64-k step of the block's
// packed words is expanded once, by all 512 lanes (two words each, 17 VALU per 8
// codes, wide_dequant's exact bf16(code * s)), into a bf16 tile in LDS that the
// four row-waves read as their A operands: each expanded word feeds the products
// of 256 rows, and a wave spends ~2 expansion VALU per product instead of ~4.
//
// MFMA formulation as in w4_gemm_wide.h: C^T = W . X^T per 32x32 tile with
// v_mfma_f32_32x32x16_bf16; lane l holds A = W[n0 + l%32][unit], B = X[m0 +
// l%32][unit] (16 bytes each, one 8-code unit), and C register e holds
// Y[m0 + l%32][n0 + 8(e/4) + 4(l/32) + e%4]. Sub-step j of a step takes unit 2j + h
// in lane half h from both operands (the same k permutation on both sides).
//
// Staging per 64-k step (one barrier per step):
//   X tile [256][64] bf16 (32 KB) and the packed words [128][32 B] plus one scale
//   dword per weight row go global -> LDS with global_load_lds (no VGPRs on the
//   way), X two steps ahead, the packed words three (3 buffers of each);
//   during step s the lanes expand step s + 1's words into the other of two bf16
//   weight tiles [128][64] while the products of step s read the first.
// Rows of every staged tile are 128 bytes; 16-byte unit u of row r sits at slot
// u ^ ((r >> 1) & 7), so each 16-lane phase of an operand read (16 consecutive
// rows, one unit) and of the expansion's stores covers the 64 banks once.
// LDS at 128 weight rows: 3 x 32 + 2 x 16 + 3 x 4.5 KB = 141.5 KB; at 192 (the
// q/k/v width of an 8B-class model: 6144 columns in 32 blocks) 2 x 32 + 2 x 24 +
// 3 x 6.75 KB = 132.25 KB; one block per CU. The 128-row forms stage [128][64] X
// tiles (16 KB) and 128, 64 or 32 weight rows (70.75 KB at 64).
#pragma once

#include "common.h"
#include "w4_gemm.h"
#include "w4_gemm_wide.h"

namespace aoto {

constexpr int kLdsBK = 64;     // k per step: four 16-k sub-steps

// Global -> LDS loads issued from inline assembly (lane l's 16 / 4 bytes land at
// lds + 16 l / 4 l; lds is wave-uniform). The compiler then tracks none of them,
// so the step's hand-counted vmcnt waits are the only ones: with the builtin, its
// wait analysis lost track of which buffer a load writes and waited for every
// load in flight before some reads and stores of other buffers.
AOTO_DEVICE uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// The address is a wave-uniform base (SGPRs) plus a 32-bit per-lane byte offset.
AOTO_DEVICE void dma16_raw(const void* base, uint32_t off, const void* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_address(lds)), "v"(off),
               "s"(base)
               : "memory", "m0");
}
AOTO_DEVICE void dma4_raw(const void* base, uint32_t off, const void* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds_address(lds)), "v"(off),
               "s"(base)
               : "memory", "m0");
}

// Byte offset of 16-byte unit u of row r in a tile of 128-byte rows.
AOTO_DEVICE int lds_unit(int r, int u) { return r * 128 + ((u ^ ((r >> 1) & 7)) << 4); }

// NW waves (8: two per SIMD, 4: one), NW / WGN along m and WGN (1 or 2) along n;
// MT 32-row tiles and NT 32-column tiles (per weight) per wave: BM = 32 MT NW / WGN
// = 256 or 128 rows, 32 WGN NT columns per weight, NP weights (2 for the paired
// gate/up) - WR = 32 NP WGN NT = 64, 128 or 192 weight rows. Per sub-step a wave
// reads MT + NP NT operands for MT NP NT products: at 8 waves (MT = 2) 4 for 4, or 5
// for 6 at NT = 3; the 128-row paired form (4 waves, WGN = 1, MT = NT = 1) 3 for 2.
// X takes three staging buffers where they fit 160 KB, else two (WR = 192 at 256
// rows: each step's X is then loaded one step ahead).
// PARTIAL (split-K, the single form): block z of the grid's third dimension takes k
// in [z kslice, min(K, (z + 1) kslice)) and stores its f32 tile to partials[z][m][n]
// (the layout the split reduce kernels of w4_gemm.h read); no epilogue.
template <int NW, int WGN, int MT, int NT, bool PAIRED, bool BIAS, bool RESIDUAL, bool PARTIAL = false>
__device__ void w4_gemm_lds_body(const uint16_t* __restrict__ X, const uint32_t* __restrict__ words,
                                 const uint16_t* __restrict__ scales, const uint32_t* __restrict__ up_words,
                                 const uint16_t* __restrict__ up_scales, const uint16_t* __restrict__ bias,
                                 const uint16_t* __restrict__ residual, uint16_t* __restrict__ Y, int M, int N,
                                 int K, int group, float* __restrict__ partials = nullptr, int kslice = 0) {
  static_assert(!(PAIRED && (BIAS || RESIDUAL)), "the paired form has its own epilogue");
  static_assert(!(PARTIAL && (PAIRED || BIAS || RESIDUAL)), "split partials carry no epilogue");
  constexpr int NP = PAIRED ? 2 : 1;
  static_assert(WGN == 1 || WGN == 2, "one or two waves along n");
  constexpr int WGM = NW / WGN;
  constexpr int BM = WGM * 32 * MT;
  constexpr int BNW = WGN * 32 * NT;  // columns per weight
  constexpr int WR = NP * BNW;                       // weight rows per block
  static_assert(WR == 32 || WR == 64 || WR == 128 || WR == 192, "32, 64, 128 or 192 weight rows per block");
  static_assert(BM == 256 || BM == 128, "256 or 128 X rows per block");
  constexpr int XT = BM * 128;                       // bytes of a staged X tile
  constexpr int XDW = XT / 1024 / NW;                // 1-KB X loads per wave and step
  constexpr int WT = WR * 128;                       // bytes of a bf16 weight tile
  constexpr int PT = WR * 32;                        // bytes of a step's packed words
  constexpr int PST = PT + WR * 4;                   // ... and their scale dwords
  constexpr int XS = 3 * XT + 2 * WT + 3 * PST <= 160 * 1024 ? 3 : 2;  // X staging buffers
  constexpr int PW = WR / NW;                        // packed rows each wave loads: 16, 24 or 32
  constexpr int UPT = WR * 8 / (64 * NW);            // words each lane expands per step: 2, 3 or 4
  static_assert(UPT >= 1 && WR % NW == 0, "every lane expands whole words");
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  static_assert(2 * PW <= 64 && UPT <= 4, "one packed-word load per wave and step");

  __shared__ __attribute__((aligned(16))) uint8_t xs0[XT];
  __shared__ __attribute__((aligned(16))) uint8_t xs1[XT];
  __shared__ __attribute__((aligned(16))) uint8_t xs2[XS == 3 ? XT : 16];
  __shared__ __attribute__((aligned(16))) uint8_t ws0[WT];
  __shared__ __attribute__((aligned(16))) uint8_t ws1[WT];
  __shared__ __attribute__((aligned(16))) uint8_t ps0[PST];  // words [128][32 B], then scales [128]
  __shared__ __attribute__((aligned(16))) uint8_t ps1[PST];
  __shared__ __attribute__((aligned(16))) uint8_t ps2[PST];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int col = lane & 31, half = lane >> 5;
  const int wm = wave / WGN, wn = wave % WGN;
  const int m_block = blockIdx.y * BM, n_block = blockIdx.x * BNW;
  const int kw = K >> 3;
  const int groups = K / group;
  const int gshift = __builtin_ctz(group);
  const int kbase = PARTIAL ? (int)blockIdx.z * kslice : 0;  // kslice % 64 == 0 (host)
  const int steps = ((PARTIAL ? min(K, kbase + kslice) : K) - kbase) / kLdsBK;

  wide_f32x16 acc[NP][NT][MT];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
      for (int u = 0; u < MT; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[p][i][u][e] = 0.f;

  // Load sources: a per-lane 32-bit byte offset from a per-step uniform base.
  // X load i of this wave: rows 8 (XDW wave + i) + lane / 8, slot lane % 8 holding
  // unit (lane % 8) ^ ((row >> 1) & 7); rows past M clamped (never stored).
  uint32_t xoff[XDW];
#pragma unroll
  for (int i = 0; i < XDW; ++i) {
    const int r = 8 * (wave * XDW + i) + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    xoff[i] = (uint32_t)(((size_t)min(m_block + r, M - 1) * K + 8 * c) * 2);
  }
  // Packed rows PW w .. PW w + PW - 1 of the block (the gate's rows, then the up's):
  // lanes below 2 PW load 16 bytes each (two per row), lanes below PW one scale dword.
  const int prow = PW * wave + (lane >> 1) % PW;
  const bool up_rows = PAIRED && PW * wave_u >= BNW;  // wave-uniform
  const int pn = min(n_block + prow % BNW, N - 1);
  const uint8_t* pbase = reinterpret_cast<const uint8_t*>(up_rows ? up_words : words);
  const uint8_t* sbase = reinterpret_cast<const uint8_t*>(up_rows ? up_scales : scales);
  const uint32_t poff = (uint32_t)(((size_t)pn * kw) * 4 + 16 * (lane & 1));
  const int srow = PW * wave + lane % PW;
  const uint32_t soff = (uint32_t)((size_t)min(n_block + srow % BNW, N - 1) * groups * 2);

  // Step st's loads (steps past the end re-read the last one).
  auto issue_x = [&](int st, uint8_t* xb) __attribute__((always_inline)) {
    const int k0 = kbase + min(st, steps - 1) * kLdsBK;
    const uint8_t* xsrc = reinterpret_cast<const uint8_t*>(X) + 2 * k0;
#pragma unroll
    for (int i = 0; i < XDW; ++i) dma16_raw(xsrc, xoff[i], xb + (wave_u * XDW + i) * 1024);
  };
  // units k0 / 8 .. + 8 of the row (4 bytes each); the scale dword holding group k0 >> gshift
  // (groups per row are even, so the aligned pair never leaves the row)
  auto issue_p = [&](int st, uint8_t* pb) __attribute__((always_inline)) {
    const int k0 = kbase + min(st, steps - 1) * kLdsBK;
    if (2 * PW == 64 || lane < 2 * PW) dma16_raw(pbase + (k0 >> 3) * 4, poff, pb + wave_u * 32 * PW);
    if (lane < PW) dma4_raw(sbase + ((k0 >> gshift) & ~1) * 2, soff, pb + PT + wave_u * 4 * PW);
  };

  // Expansion: thread t takes unit t % 8 of weight rows t / 8 + 8 NW v, v < UPT.
  const int du = t & 7;
  int dwr[UPT];
#pragma unroll
  for (int v = 0; v < UPT; ++v) dwr[v] = lds_unit((t >> 3) + 8 * NW * v, du);
  const WideMasks km = wide_masks<4>();
  uint32_t dword[UPT], dscale[UPT];
  auto expand_read = [&](const uint8_t* pb) __attribute__((always_inline)) {
#pragma unroll
    for (int v = 0; v < UPT; ++v) {
      const int r = (t >> 3) + 8 * NW * v;
      dword[v] = *reinterpret_cast<const uint32_t*>(pb + r * 32 + 4 * du);
      dscale[v] = *reinterpret_cast<const uint32_t*>(pb + PT + 4 * r);
    }
  };
  // the scale of this thread's unit: group 32 -> group du / 4 of the step's pair;
  // larger -> the step's group, the low or high half of its aligned pair
  auto expand = [&](int v, int st) __attribute__((always_inline)) {
    const int k0 = kbase + min(st, steps - 1) * kLdsBK;
    const int hsel = group == 32 ? (du >> 2) : ((k0 >> gshift) & 1);
    const float s = bf16_to_f32((dscale[v] >> (16 * hsel)) & 0xFFFFu);
    return wide_dequant(dword[v], wide_scale<4>(s), km);
  };

  // Operand reads: A (p, i) = weight row p BNW + 32 (NT wn + i) + col, B (u) = X row
  // 32 (MT wm + u) + col; every such row has the same swizzle as its first, so
  // sub-step j's unit 2j + h is base ^ (32 j) and the tiles are immediate offsets.
  const int ar = 32 * NT * wn + col, br = 32 * MT * wm + col;
  const int aoff = ar * 128 + ((half ^ ((ar >> 1) & 7)) << 4);
  const int boff = br * 128 + ((half ^ ((br >> 1) & 7)) << 4);
  bf16x8_v a[2][NP][NT], b[2][MT];
  auto read_ops = [&](auto into_c, auto j_c, const uint8_t* wb, const uint8_t* xb) __attribute__((always_inline)) {
    constexpr int into = decltype(into_c)::value, j = decltype(j_c)::value;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int i = 0; i < NT; ++i)
        a[into][p][i] = *reinterpret_cast<const bf16x8_v*>(wb + ((aoff ^ (32 * j)) + (p * BNW + 32 * i) * 128));
#pragma unroll
    for (int u = 0; u < MT; ++u)
      b[into][u] = *reinterpret_cast<const bf16x8_v*>(xb + ((boff ^ (32 * j)) + 32 * u * 128));
  };
  auto products = [&](auto from_c) __attribute__((always_inline)) {
    constexpr int from = decltype(from_c)::value;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int u = 0; u < MT; ++u)
          acc[p][i][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[from][p][i], b[from][u], acc[p][i][u], 0, 0, 0);
  };
  constexpr int DPS = XDW + 2;  // a wave's loads per step

  // Step s: issue step s + XS - 1's X and step s + 3's words; expand step s + 1's
  // words (read at the start, stored over the sub-steps) while the products of
  // step s run; wait for step s + 1's X and step s + 2's words, barrier, read
  // sub-step 0's operands of step s + 1.
  auto step = [&](int s, const uint8_t* xc, const uint8_t* wc, uint8_t* wn_, const uint8_t* pd, uint8_t* xi,
                  uint8_t* pi, const uint8_t* xn) __attribute__((always_inline)) {
    issue_x(s + XS - 1, xi);
    issue_p(s + 3, pi);
    expand_read(pd);
    // word v is expanded in sub-step ex(v) and stored in the next (the last in the last)
    bf16x8_v e[UPT];
    static_for<4>([&](auto j_c) __attribute__((always_inline)) {
      constexpr int j = decltype(j_c)::value;
      using Cur = std::integral_constant<int, j & 1>;
      using Nxt = std::integral_constant<int, 1 - (j & 1)>;
      if constexpr (j < 3) read_ops(Nxt{}, std::integral_constant<int, j + 1>{}, wc, xc);
      products(Cur{});
      static_for<UPT>([&](auto v_c) __attribute__((always_inline)) {
        constexpr int v = decltype(v_c)::value;
        constexpr int ex = UPT == 4 ? v : v + 1;
        constexpr int st = ex + 1 < 4 ? ex + 1 : 3;
        if constexpr (st == j && st != ex) *reinterpret_cast<bf16x8_v*>(wn_ + dwr[v]) = e[v];
      });
      static_for<UPT>([&](auto v_c) __attribute__((always_inline)) {
        constexpr int v = decltype(v_c)::value;
        constexpr int ex = UPT == 4 ? v : v + 1;
        constexpr int st = ex + 1 < 4 ? ex + 1 : 3;
        if constexpr (ex == j) e[v] = expand(v, s + 1);
        if constexpr (ex == j && st == ex) *reinterpret_cast<bf16x8_v*>(wn_ + dwr[v]) = e[v];
      });
      __builtin_amdgcn_sched_barrier(0);
    });
    // step s + 1's X and step s + 2's words are in (with two X buffers step s + 1's X
    // went out at this step's start, ahead of its words)
    AOTO_WAIT_VMCNT(XS == 3 ? DPS : 2);
    AOTO_WAIT_LGKMCNT(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");  // no LDS access moves across the barrier
    read_ops(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, wn_, xn);
  };

  // Prologue: X 0 (and 1 with three buffers), words 0, 1 and 2 in flight; step 0's
  // words expanded; step 1's words in; sub-step 0's operands of step 0 read.
  issue_x(0, xs0);
  issue_p(0, ps0);
  if constexpr (XS == 3) issue_x(1, xs1);
  issue_p(1, ps1);
  issue_p(2, ps2);
  AOTO_WAIT_VMCNT(XS == 3 ? DPS + 2 : 4);  // X 0 and words 0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  expand_read(ps0);
#pragma unroll
  for (int v = 0; v < UPT; ++v) *reinterpret_cast<bf16x8_v*>(ws0 + dwr[v]) = expand(v, 0);
  AOTO_WAIT_VMCNT(2);  // (X 1 and) words 1
  AOTO_WAIT_LGKMCNT(0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  read_ops(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, ws0, xs0);

  // Six steps per trip (X in XS buffers, words in 3, weight tiles in 2), then the
  // remaining steps % 6.
  auto step6 = [&](auto i_c, int s) __attribute__((always_inline)) {
    constexpr int i = decltype(i_c)::value;
    auto X3 = [&](auto b_c) __attribute__((always_inline)) -> uint8_t* {
      constexpr int b = decltype(b_c)::value % XS;
      if constexpr (b == 0) return xs0; else if constexpr (b == 1) return xs1; else return xs2;
    };
    auto P3 = [&](auto b_c) __attribute__((always_inline)) -> uint8_t* {
      constexpr int b = decltype(b_c)::value % 3;
      if constexpr (b == 0) return ps0; else if constexpr (b == 1) return ps1; else return ps2;
    };
    auto W2 = [&](auto b_c) __attribute__((always_inline)) -> uint8_t* {
      if constexpr (decltype(b_c)::value % 2 == 0) return ws0; else return ws1;
    };
    using I0 = std::integral_constant<int, i>;
    using I1 = std::integral_constant<int, i + 1>;
    using IX = std::integral_constant<int, i + XS - 1>;
    step(s, X3(I0{}), W2(I0{}), W2(I1{}), P3(I1{}), X3(IX{}), P3(I0{}), X3(I1{}));
  };
  int s = 0;
  for (; s + 6 <= steps; s += 6) {
    step6(std::integral_constant<int, 0>{}, s);
    step6(std::integral_constant<int, 1>{}, s + 1);
    step6(std::integral_constant<int, 2>{}, s + 2);
    step6(std::integral_constant<int, 3>{}, s + 3);
    step6(std::integral_constant<int, 4>{}, s + 4);
    step6(std::integral_constant<int, 5>{}, s + 5);
  }
  const int rest = steps - s;
  if (rest > 0) {
    step6(std::integral_constant<int, 0>{}, s);
    if (rest > 1) {
      step6(std::integral_constant<int, 1>{}, s + 1);
      if (rest > 2) {
        step6(std::integral_constant<int, 2>{}, s + 2);
        if (rest > 3) {
          step6(std::integral_constant<int, 3>{}, s + 3);
          if (rest > 4) step6(std::integral_constant<int, 4>{}, s + 4);
        }
      }
    }
  }
  // The last steps' loads (past the end: re-reads of the last step) still land in
  // LDS: wait for them before the epilogue reuses the X buffers.
  AOTO_WAIT_VMCNT(0);
  __syncthreads();

  // Epilogue: each 32 x 32 sub-tile through the wave's own 4.5-KB LDS slot (f32
  // rows 144 bytes apart), read back eight lanes per row: 64 contiguous bytes of
  // residual and output per row.
  constexpr int SLOTS = XT / 4608;  // epilogue slots per X buffer: 7 at 256 rows, 3 at 128
  static_assert(NW <= 2 * SLOTS, "a slot per wave in the first two X buffers");
  float* slot = reinterpret_cast<float*>((wave < SLOTS ? xs0 : xs1) + (wave % SLOTS) * 4608);
  const int m_wave = m_block + 32 * MT * wm;
  if constexpr (PARTIAL) {
    float* part = partials + (size_t)blockIdx.z * M * N;
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const int n = n_block + 32 * (NT * wn + i) + 4 * (lane & 7);
#pragma unroll
      for (int u = 0; u < MT; ++u) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<float4*>(slot + col * 36 + 8 * g + 4 * half) =
              make_float4(acc[0][i][u][4 * g], acc[0][i][u][4 * g + 1], acc[0][i][u][4 * g + 2],
                          acc[0][i][u][4 * g + 3]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = (lane >> 3) + 8 * q;
          const int m = m_wave + 32 * u + r;
          const float4 f = *reinterpret_cast<const float4*>(slot + r * 36 + 4 * (lane & 7));
          if (m < M && n < N) *reinterpret_cast<float4*>(part + (size_t)m * N + n) = f;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const int n0 = n_block + 32 * (NT * wn + i);
    float4 bcol = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (BIAS) {
      const uint2 bb = *reinterpret_cast<const uint2*>(bias + min(n0 + 4 * (lane & 7), N - 4));
      bcol = make_float4(bf16_lo(bb.x), bf16_hi(bb.x), bf16_lo(bb.y), bf16_hi(bb.y));
    }
#pragma unroll
    for (int u = 0; u < MT; ++u) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float v[4] = {acc[0][i][u][4 * g], acc[0][i][u][4 * g + 1], acc[0][i][u][4 * g + 2], acc[0][i][u][4 * g + 3]};
        if constexpr (PAIRED) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float gt = round_bf16(v[e]);
            v[e] = acc[NP - 1][i][u][4 * g + e] * (gt / (1.0f + expf(-gt)));
          }
        }
        *reinterpret_cast<float4*>(slot + col * 36 + 8 * g + 4 * half) = make_float4(v[0], v[1], v[2], v[3]);
      }
      const int n = n0 + 4 * (lane & 7);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = (lane >> 3) + 8 * q;
        const int m = m_wave + 32 * u + r;
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
        *reinterpret_cast<uint2*>(Y + (size_t)m * N + n) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
    }
  }
}

}  // namespace aoto

// aoto_w4_gemm_d{NW}w{MT}x{NT}_b{BIAS}_r{RES}: 256-row blocks of NW waves, two along n.
#define AOTO_GEMM_LDS_INSTANCE(NW, MT, NT, BIAS, RES)                                                         \
  extern "C" __global__ __launch_bounds__(64 * NW, 1) void aoto_w4_gemm_d##NW##w##MT##x##NT##_b##BIAS##_r##RES( \
      const uint16_t* X, const uint32_t* words, const uint16_t* scales, const uint16_t* bias,                 \
      const uint16_t* residual, uint16_t* Y, int M, int N, int K, int group) {                                \
    aoto::w4_gemm_lds_body<NW, 2, MT, NT, false, BIAS, RES>(X, words, scales, nullptr, nullptr, bias, residual, \
                                                            Y, M, N, K, group);                              \
  }
// aoto_w4_gemm_d{NW}w{MT}x{NT}_paired: the MLP's gate/up pair, two waves along n
// (256 x (64 + 64) blocks at NW = 8, MT = 2; 128 x (64 + 64) at NW = 4, MT = 2).
#define AOTO_GEMM_LDS_PAIRED_INSTANCE(NW, MT, NT)                                                             \
  extern "C" __global__ __launch_bounds__(64 * NW, 1) void aoto_w4_gemm_d##NW##w##MT##x##NT##_paired(          \
      const uint16_t* X, const uint32_t* words, const uint16_t* scales, const uint32_t* up_words,             \
      const uint16_t* up_scales, uint16_t* Y, int M, int N, int K, int group) {                               \
    aoto::w4_gemm_lds_body<NW, 2, MT, NT, true, false, false>(X, words, scales, up_words, up_scales, nullptr,   \
                                                              nullptr, Y, M, N, K, group);                   \
  }
// aoto_w4_gemm_d{NW}c{WGN}w{MT}x{NT}_split: the single form's split-K partials (f32
// partials[z][m][n], k slice z of kslice), for short prompts whose column blocks alone
// do not fill the chip; a reduce kernel applies the epilogue.
#define AOTO_GEMM_LDS_SPLIT_INSTANCE(NW, WGN, MT, NT)                                                         \
  extern "C" __global__ __launch_bounds__(64 * NW, 1) void aoto_w4_gemm_d##NW##c##WGN##w##MT##x##NT##_split(   \
      const uint16_t* X, const uint32_t* words, const uint16_t* scales, float* partials, int M, int N, int K, \
      int group, int kslice) {                                                                                \
    aoto::w4_gemm_lds_body<NW, WGN, MT, NT, false, false, false, true>(                                       \
        X, words, scales, nullptr, nullptr, nullptr, nullptr, nullptr, M, N, K, group, partials, kslice);     \
  }
// aoto_w4_gemm_d{NW}c1w{MT}x{NT}_paired: the same with one wave along n (at NW = 4,
// MT = NT = 1: 128 x (32 + 32) blocks, twice the blocks of the 64-column form for
// short prompts).
#define AOTO_GEMM_LDS_PAIRED_COLUMN_INSTANCE(NW, MT, NT)                                                      \
  extern "C" __global__ __launch_bounds__(64 * NW, 1) void aoto_w4_gemm_d##NW##c1w##MT##x##NT##_paired(       \
      const uint16_t* X, const uint32_t* words, const uint16_t* scales, const uint32_t* up_words,             \
      const uint16_t* up_scales, uint16_t* Y, int M, int N, int K, int group) {                               \
    aoto::w4_gemm_lds_body<NW, 1, MT, NT, true, false, false>(X, words, scales, up_words, up_scales, nullptr,   \
                                                              nullptr, Y, M, N, K, group);                   \
  }
