// Device helpers shared by every gfx950 kernel of the W4 decoder path.
//
// bf16 values travel as raw uint16 bit patterns; all arithmetic is f32 and every
// store rounds once, to nearest-even, which is the cast torch and MLX perform.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

#define AOTO_DEVICE __device__ __forceinline__

AOTO_DEVICE float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
AOTO_DEVICE float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
AOTO_DEVICE float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xFFFF0000u); }

// Round-to-nearest-even f32 -> bf16 bits; NaN stays a quiet NaN.
AOTO_DEVICE uint32_t f32_to_bf16(float value) {
  uint32_t u = __float_as_uint(value);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

AOTO_DEVICE float round_bf16(float value) { return bf16_to_f32(f32_to_bf16(value)); }

AOTO_DEVICE uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
}

// The same two roundings in one v_cvt_pk_bf16_f32 (round to nearest even; for
// every non-NaN f32 input the bits equal pack_bf16x2's - checked on gfx950 over
// all 2^32 patterns; a NaN may keep a different payload).
AOTO_DEVICE uint32_t cvt_pk_bf16(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Two bf16 products accumulated into f32: acc + a.lo*b.lo + a.hi*b.hi.
AOTO_DEVICE float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                        __builtin_bit_cast(bf16x2_t, b), acc, false);
}

// Cross-lane moves inside 16-lane rows through DPP (a VALU operand modifier, no
// LDS round trip): quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2),
// row_half_mirror (quads 0<->1 of each 8), row_mirror (halves of each 16).
template <int CTRL>
AOTO_DEVICE float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

// The pair {value of lane l & ~16, value of lane l | 16} (permlane16_swap of a
// register with itself: rows 0/1 and 2/3 exchange) and the same across the
// wave's halves (permlane32_swap): lane l ^ 16 / l ^ 32 without an LDS round
// trip. Lane layout checked on gfx950.
AOTO_DEVICE float xor16_sum(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
AOTO_DEVICE float xor32_sum(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
AOTO_DEVICE float xor16_max(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
AOTO_DEVICE float xor32_max(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// Sum over the `WIDTH` lanes of an aligned lane group (WIDTH a power of two <=
// 64); every lane of the group gets the total. Up to 16 lanes it is four DPP
// steps; wider groups add permlane swaps across rows and halves. Each step adds
// a lane's value and its partner's (l ^ 1, 2, 4 or 8 by DPP, then l ^ 16, 32).
template <int WIDTH>
AOTO_DEVICE float group_sum(float value) {
  if (WIDTH >= 2) value += dpp_move<kDppXor1>(value);
  if (WIDTH >= 4) value += dpp_move<kDppXor2>(value);
  if (WIDTH >= 8) value += dpp_move<kDppHalfMirror>(value);
  if (WIDTH >= 16) value += dpp_move<kDppMirror>(value);
  if (WIDTH >= 32) value = xor16_sum(value);
  if (WIDTH >= 64) value = xor32_sum(value);
  return value;
}

template <int WIDTH>
AOTO_DEVICE float group_max(float value) {
  if (WIDTH >= 2) value = fmaxf(value, dpp_move<kDppXor1>(value));
  if (WIDTH >= 4) value = fmaxf(value, dpp_move<kDppXor2>(value));
  if (WIDTH >= 8) value = fmaxf(value, dpp_move<kDppHalfMirror>(value));
  if (WIDTH >= 16) value = fmaxf(value, dpp_move<kDppMirror>(value));
  if (WIDTH >= 32) value = xor16_max(value);
  if (WIDTH >= 64) value = xor32_max(value);
  return value;
}

// Whole-wave sum / max returned uniformly: DPP within the four 16-lane rows,
// then the four row results read with v_readlane.
AOTO_DEVICE float wave_sum(float value) {
  value = group_sum<16>(value);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 0)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 16)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 32)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 48));
}

AOTO_DEVICE float wave_max(float value) {
  value = group_max<16>(value);
  return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 0)),
                     __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 16))),
               fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 32)),
                     __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), 48))));
}

// Block-wide sum over a block of THREADS threads (a multiple of 64, at most
// 1024); every thread gets the total. `scratch` needs one float per wave.
// Contains a barrier: call from all threads. The thread count is a template
// argument because reading blockDim costs a memory round trip.
template <int THREADS>
AOTO_DEVICE float block_sum(float value, float* scratch) {
  value = wave_sum(value);
  const int wave = threadIdx.x >> 6;
  constexpr int waves = THREADS / 64;
  if ((threadIdx.x & 63) == 0) scratch[wave] = value;
  __syncthreads();
  float total = 0.f;
  for (int w = 0; w < waves; ++w) total += scratch[w];
  __syncthreads();
  return total;
}

// Order-preserving key of a bf16 value with the index in the low bits so that
// the maximum key is the largest value and, among equal values, the first index.
// NaN never wins.
AOTO_DEVICE unsigned long long argmax_key(uint32_t bits16, int index) {
  uint32_t u = bits16 & 0xFFFFu;
  u = (u & 0x8000u) ? (~u & 0xFFFFu) : (u | 0x8000u);
  if ((bits16 & 0x7FFFu) > 0x7F80u) u = 0;
  return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)index);
}

// Index encoded in an argmax key.
AOTO_DEVICE long long argmax_key_index(unsigned long long key) {
  return (long long)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
}

AOTO_DEVICE unsigned long long max_u64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

// Whole-wave maximum of a 64-bit key, every lane gets it: the two halves move
// together through the same DPP steps as group_max, then permlane swaps across
// rows and halves (no LDS round trip).
template <int CTRL>
AOTO_DEVICE unsigned long long dpp_move_u64(unsigned long long v) {
  const uint32_t lo = __builtin_amdgcn_update_dpp(0u, (uint32_t)v, CTRL, 0xF, 0xF, false);
  const uint32_t hi = __builtin_amdgcn_update_dpp(0u, (uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  return ((unsigned long long)hi << 32) | lo;
}
AOTO_DEVICE unsigned long long wave_max_u64(unsigned long long v) {
  v = max_u64(v, dpp_move_u64<kDppXor1>(v));
  v = max_u64(v, dpp_move_u64<kDppXor2>(v));
  v = max_u64(v, dpp_move_u64<kDppHalfMirror>(v));
  v = max_u64(v, dpp_move_u64<kDppMirror>(v));
  {
    const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
    v = max_u64(((unsigned long long)hi[0] << 32) | lo[0], ((unsigned long long)hi[1] << 32) | lo[1]);
  }
  {
    const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
    v = max_u64(((unsigned long long)hi[0] << 32) | lo[0], ((unsigned long long)hi[1] << 32) | lo[1]);
  }
  return v;
}
