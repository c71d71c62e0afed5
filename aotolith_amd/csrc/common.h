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

// Two bf16 products accumulated into f32: acc + a.lo*b.lo + a.hi*b.hi.
AOTO_DEVICE float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                        __builtin_bit_cast(bf16x2_t, b), acc, false);
}

// Sum over the `width` lanes of an aligned lane group (width a power of two <= 64).
template <int WIDTH>
AOTO_DEVICE float group_sum(float value) {
#pragma unroll
  for (int offset = WIDTH / 2; offset > 0; offset >>= 1) value += __shfl_xor(value, offset, 64);
  return value;
}

template <int WIDTH>
AOTO_DEVICE float group_max(float value) {
#pragma unroll
  for (int offset = WIDTH / 2; offset > 0; offset >>= 1) value = fmaxf(value, __shfl_xor(value, offset, 64));
  return value;
}

// Block-wide sum for blocks of up to 1024 threads; every thread gets the total.
// `scratch` needs one float per wave. Contains a barrier: call from all threads.
AOTO_DEVICE float block_sum(float value, float* scratch) {
  value = group_sum<64>(value);
  const int wave = threadIdx.x >> 6;
  const int waves = (blockDim.x + 63) >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = value;
  __syncthreads();
  float total = 0.f;
  for (int w = 0; w < waves; ++w) total += scratch[w];
  __syncthreads();
  return total;
}
