// Symmetric int4 group quantizer/packer and the bf16 unpack, on the GPU.
//
// Bit-exact restatement of quantize.py:95-152 and models/quantized.py:61-76,
// 133-163 of the reference:
//   scale = max|w| / 7 in f32 (an all-zero group takes 1/7);
//   code  = clip(rint(w / scale), -8, 7) with IEEE f32 division, half-to-even;
//   word j of a row holds codes 8j..8j+7, code 8j+k at bits 4k;
//   the stored scale is bf16(scale) (RNE) while the codes use the f32 scale.
// The unpack writes bf16(code * scale_bf16), the torch op's value in bf16.
#pragma once

#include "common.h"

// One thread per (row, group). `src_f32` selects an f32 source, else bf16.
extern "C" __global__ __launch_bounds__(256) void aoto_w4_quantize(
    const void* __restrict__ src, int src_f32, int rows, int inner, int group,
    int32_t* __restrict__ packed, uint16_t* __restrict__ scales_bf16, float* __restrict__ scales_f32) {
  const int groups = inner / group;
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long long)rows * groups) return;
  const int row = (int)(gid / groups);
  const int g = (int)(gid - (long long)row * groups);
  const size_t base = (size_t)row * inner + (size_t)g * group;
  auto load = [&](int i) -> float {
    if (src_f32) return reinterpret_cast<const float*>(src)[base + i];
    return bf16_to_f32(reinterpret_cast<const uint16_t*>(src)[base + i]);
  };
  float widest = 0.f;
  for (int i = 0; i < group; ++i) widest = fmaxf(widest, fabsf(load(i)));
  const float scale = (widest > 0.f ? widest : 1.0f) / 7.0f;
  int32_t* out = packed + (size_t)row * (inner >> 3) + (size_t)g * (group >> 3);
  for (int w = 0; w < (group >> 3); ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float code = rintf(load(w * 8 + k) / scale);
      code = fminf(fmaxf(code, -8.0f), 7.0f);
      word |= ((uint32_t)(int)code & 0xFu) << (4 * k);
    }
    out[w] = (int32_t)word;
  }
  scales_bf16[(size_t)row * groups + g] = (uint16_t)f32_to_bf16(scale);
  if (scales_f32) scales_f32[(size_t)row * groups + g] = scale;
}

// One thread per packed word: eight bf16(code * scale) values, one 16-byte store.
extern "C" __global__ __launch_bounds__(256) void aoto_w4_dequantize(
    const int32_t* __restrict__ packed, const uint16_t* __restrict__ scales, int rows, int inner,
    int group, uint16_t* __restrict__ out) {
  const int words = inner >> 3;
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long long)rows * words) return;
  const int row = (int)(gid / words);
  const int w = (int)(gid - (long long)row * words);
  const uint32_t word = (uint32_t)packed[gid];
  const float s = bf16_to_f32(scales[(size_t)row * (inner / group) + (w * 8) / group]);
  uint32_t v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int code = (int)(word << (28 - 4 * k)) >> 28;
    v[k] = f32_to_bf16((float)code * s);
  }
  uint4 o;
  o.x = v[0] | (v[1] << 16);
  o.y = v[2] | (v[3] << 16);
  o.z = v[4] | (v[5] << 16);
  o.w = v[6] | (v[7] << 16);
  reinterpret_cast<uint4*>(out)[gid] = o;
}
