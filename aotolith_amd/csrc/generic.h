// Generic graph kernels for the compile_callable / compile_module plans.
//
// A captured graph (torch.export + core-ATen decompositions, see
// aotolith_amd/graph.py) is lowered node by node onto a small set of kernels:
// strided elementwise (unary / binary / where, with broadcasting and element
// type conversion), row reductions and scans, a strided batched GEMM, advanced
// indexing (embedding / index), strided copies (clone, cat, contiguous), fills
// and aranges, and two fused legalized patterns, the HF RMSNorm chain and
// scaled-dot-product attention. This mirrors what the reference's mlx-reference
// target executes per node (runtime/mlx_ops/__init__.py:239-620) without its
// per-op MLX dispatch: every node is one gfx950 launch.
//
// These kernels serve generality (any static-shape module), not the decoder's
// hot path: they favour simple, always-in-bounds index arithmetic over speed.
// Every op reads through element strides, so views (permute, expand, slice,
// unsqueeze) never copy.
#pragma once

#include "aoto_hip.h"
#include "common.h"
#include "generic_args.h"

namespace aoto {

constexpr int kGenThreads = 256;

AOTO_DEVICE double load_value(const void* p, int dtype, long long off) {
  switch (dtype) {
    case AOTO_DT_F32: return (double)static_cast<const float*>(p)[off];
    case AOTO_DT_BF16: return (double)bf16_to_f32(static_cast<const uint16_t*>(p)[off]);
    case AOTO_DT_I64: return (double)static_cast<const long long*>(p)[off];
    case AOTO_DT_I32: return (double)static_cast<const int*>(p)[off];
    case AOTO_DT_BOOL:
    case AOTO_DT_U8: return (double)static_cast<const uint8_t*>(p)[off];
    case AOTO_DT_I8: return (double)static_cast<const int8_t*>(p)[off];
    default: return 0.0;
  }
}

AOTO_DEVICE long long load_int(const void* p, int dtype, long long off) {
  switch (dtype) {
    case AOTO_DT_I64: return static_cast<const long long*>(p)[off];
    case AOTO_DT_I32: return static_cast<const int*>(p)[off];
    case AOTO_DT_BOOL:
    case AOTO_DT_U8: return static_cast<const uint8_t*>(p)[off];
    case AOTO_DT_I8: return static_cast<const int8_t*>(p)[off];
    case AOTO_DT_F32: return (long long)static_cast<const float*>(p)[off];
    case AOTO_DT_BF16: return (long long)bf16_to_f32(static_cast<const uint16_t*>(p)[off]);
    default: return 0;
  }
}

// Store a float result (rounded once to the element type; float -> int truncates).
AOTO_DEVICE void store_float(void* p, int dtype, long long off, float v) {
  switch (dtype) {
    case AOTO_DT_F32: static_cast<float*>(p)[off] = v; break;
    case AOTO_DT_BF16: static_cast<uint16_t*>(p)[off] = (uint16_t)f32_to_bf16(v); break;
    case AOTO_DT_I64: static_cast<long long*>(p)[off] = (long long)v; break;
    case AOTO_DT_I32: static_cast<int*>(p)[off] = (int)v; break;
    case AOTO_DT_BOOL: static_cast<uint8_t*>(p)[off] = v != 0.f; break;
    case AOTO_DT_U8: static_cast<uint8_t*>(p)[off] = (uint8_t)(int)v; break;
    case AOTO_DT_I8: static_cast<int8_t*>(p)[off] = (int8_t)(int)v; break;
    default: break;
  }
}

// Store an exact value held in a double (a select / copy of any element type).
AOTO_DEVICE void store_double(void* p, int dtype, long long off, double v) {
  switch (dtype) {
    case AOTO_DT_F32: static_cast<float*>(p)[off] = (float)v; break;
    case AOTO_DT_BF16: static_cast<uint16_t*>(p)[off] = (uint16_t)f32_to_bf16((float)v); break;
    case AOTO_DT_I64: static_cast<long long*>(p)[off] = (long long)v; break;
    case AOTO_DT_I32: static_cast<int*>(p)[off] = (int)(long long)v; break;
    case AOTO_DT_BOOL: static_cast<uint8_t*>(p)[off] = v != 0.0; break;
    case AOTO_DT_U8: static_cast<uint8_t*>(p)[off] = (uint8_t)(long long)v; break;
    case AOTO_DT_I8: static_cast<int8_t*>(p)[off] = (int8_t)(long long)v; break;
    default: break;
  }
}

AOTO_DEVICE void store_int(void* p, int dtype, long long off, long long v) {
  switch (dtype) {
    case AOTO_DT_I64: static_cast<long long*>(p)[off] = v; break;
    case AOTO_DT_I32: static_cast<int*>(p)[off] = (int)v; break;
    case AOTO_DT_BOOL: static_cast<uint8_t*>(p)[off] = v != 0; break;
    case AOTO_DT_U8: static_cast<uint8_t*>(p)[off] = (uint8_t)v; break;
    case AOTO_DT_I8: static_cast<int8_t*>(p)[off] = (int8_t)v; break;
    case AOTO_DT_F32: static_cast<float*>(p)[off] = (float)v; break;
    case AOTO_DT_BF16: static_cast<uint16_t*>(p)[off] = (uint16_t)f32_to_bf16((float)v); break;
    default: break;
  }
}

AOTO_DEVICE double operand_value(const Operand& o, long long off) {
  return o.data ? load_value(o.data, o.dtype, off) : o.value;
}

AOTO_DEVICE long long operand_int(const Operand& o, long long off) {
  return o.data ? load_int(o.data, o.dtype, off) : (long long)o.value;
}

// torch's pow(x, scalar) special cases (x*x for 2, sqrt for 0.5, ...), else powf.
AOTO_DEVICE float pow_f32(float x, float e) {
  if (e == 2.f) return x * x;
  if (e == 1.f) return x;
  if (e == 3.f) return x * x * x;
  if (e == 0.5f) return sqrtf(x);
  if (e == -0.5f) return 1.0f / sqrtf(x);
  if (e == -1.f) return 1.0f / x;
  if (e == -2.f) return 1.0f / (x * x);
  if (e == 0.f) return 1.f;
  return powf(x, e);
}

AOTO_DEVICE float unary_f32(int op, float x) {
  switch (op) {
    case AOTO_EW_CAST: return x;
    case AOTO_EW_NEG: return -x;
    case AOTO_EW_ABS: return fabsf(x);
    case AOTO_EW_RECIPROCAL: return 1.0f / x;
    case AOTO_EW_SQRT: return sqrtf(x);
    case AOTO_EW_RSQRT: return 1.0f / sqrtf(x);
    case AOTO_EW_EXP: return expf(x);
    case AOTO_EW_LOG: return logf(x);
    case AOTO_EW_SIGMOID: return 1.0f / (1.0f + expf(-x));
    case AOTO_EW_SILU: return x / (1.0f + expf(-x));
    case AOTO_EW_TANH: return tanhf(x);
    case AOTO_EW_COS: return cosf(x);
    case AOTO_EW_SIN: return sinf(x);
    case AOTO_EW_RELU: return x > 0.f ? x : 0.f;
    case AOTO_EW_GELU: return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
    case AOTO_EW_GELU_TANH: {
      const float inner = 0.79788456080286536f * (x + 0.044715f * x * x * x);
      return 0.5f * x * (1.0f + tanhf(inner));
    }
    case AOTO_EW_ERF: return erff(x);
    case AOTO_EW_FLOOR: return floorf(x);
    case AOTO_EW_CEIL: return ceilf(x);
    case AOTO_EW_LOG1P: return log1pf(x);
    case AOTO_EW_EXPM1: return expm1f(x);
    default: return x;
  }
}

AOTO_DEVICE float binary_f32(int op, float a, float b, float alpha) {
  switch (op) {
    case AOTO_EW_ADD: return alpha == 1.f ? a + b : a + alpha * b;
    case AOTO_EW_SUB: return alpha == 1.f ? a - b : a - alpha * b;
    case AOTO_EW_MUL: return a * b;
    case AOTO_EW_DIV: return a / b;
    case AOTO_EW_DIV_TRUNC: return truncf(a / b);
    case AOTO_EW_DIV_FLOOR: return floorf(a / b);
    case AOTO_EW_POW: return pow_f32(a, b);
    case AOTO_EW_MAXIMUM: return (a != a || b != b) ? a + b : fmaxf(a, b);
    case AOTO_EW_MINIMUM: return (a != a || b != b) ? a + b : fminf(a, b);
    case AOTO_EW_REMAINDER: {
      const float r = fmodf(a, b);
      return (r != 0.f && ((r < 0.f) != (b < 0.f))) ? r + b : r;
    }
    default: return 0.f;
  }
}

AOTO_DEVICE long long floor_div_i64(long long a, long long b) {
  if (b == 0) return 0;
  long long q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}

AOTO_DEVICE long long int_op(int op, long long a, long long b, long long alpha) {
  switch (op) {
    case AOTO_EW_CAST: return a;
    case AOTO_EW_NEG: return -a;
    case AOTO_EW_ABS: return a < 0 ? -a : a;
    case AOTO_EW_LOGICAL_NOT: return a == 0;
    case AOTO_EW_BITWISE_NOT: return ~a;
    case AOTO_EW_ADD: return a + alpha * b;
    case AOTO_EW_SUB: return a - alpha * b;
    case AOTO_EW_MUL: return a * b;
    case AOTO_EW_DIV_TRUNC: return b == 0 ? 0 : a / b;
    case AOTO_EW_DIV_FLOOR: return floor_div_i64(a, b);
    case AOTO_EW_MAXIMUM: return a > b ? a : b;
    case AOTO_EW_MINIMUM: return a < b ? a : b;
    case AOTO_EW_REMAINDER: {
      if (b == 0) return 0;
      const long long r = a % b;
      return (r != 0 && ((r < 0) != (b < 0))) ? r + b : r;
    }
    case AOTO_EW_BIT_AND: return a & b;
    case AOTO_EW_BIT_OR: return a | b;
    case AOTO_EW_BIT_XOR: return a ^ b;
    case AOTO_EW_LOG_AND: return (a != 0) && (b != 0);
    case AOTO_EW_LOG_OR: return (a != 0) || (b != 0);
    default: return 0;
  }
}

AOTO_DEVICE bool compare_op(int op, double a, double b) {
  switch (op) {
    case AOTO_EW_EQ: return a == b;
    case AOTO_EW_NE: return a != b;
    case AOTO_EW_LT: return a < b;
    case AOTO_EW_LE: return a <= b;
    case AOTO_EW_GT: return a > b;
    case AOTO_EW_GE: return a >= b;
    case AOTO_EW_ISNAN: return a != a;
    default: return false;
  }
}

extern "C" __global__ __launch_bounds__(kGenThreads) void aoto_generic_elementwise(EwArgs a) {
  const long long stride = (long long)gridDim.x * kGenThreads;
  for (long long i = (long long)blockIdx.x * kGenThreads + threadIdx.x; i < a.total; i += stride) {
    long long rem = i, off0 = 0, off1 = 0, off2 = 0;
    for (int d = a.ndim - 1; d >= 0; --d) {
      const long long c = rem % a.shape[d];
      rem /= a.shape[d];
      off0 += c * a.in[0].strides[d];
      off1 += c * a.in[1].strides[d];
      off2 += c * a.in[2].strides[d];
    }
    if (a.domain == 0) {
      const float x = (float)operand_value(a.in[0], off0);
      float r;
      if (a.op < AOTO_EW_ADD) {
        r = unary_f32(a.op, x);
      } else {
        r = binary_f32(a.op, x, (float)operand_value(a.in[1], off1), (float)a.alpha);
      }
      store_float(a.out, a.out_dtype, i, r);
    } else if (a.domain == 1) {
      const long long x = operand_int(a.in[0], off0);
      const long long y = a.op >= AOTO_EW_ADD ? operand_int(a.in[1], off1) : 0;
      store_int(a.out, a.out_dtype, i, int_op(a.op, x, y, (long long)a.alpha));
    } else if (a.domain == 2) {
      const double x = operand_value(a.in[0], off0);
      const double y = a.op == AOTO_EW_ISNAN ? 0.0 : operand_value(a.in[1], off1);
      static_cast<uint8_t*>(a.out)[i] = compare_op(a.op, x, y) ? 1 : 0;
    } else {
      // where(cond, x, y): the selected value is copied exactly
      const bool c = operand_value(a.in[0], off0) != 0.0;
      store_double(a.out, a.out_dtype, i, c ? operand_value(a.in[1], off1) : operand_value(a.in[2], off2));
    }
  }
}

// Block-wide reductions over kGenThreads threads (scratch: one slot per wave).
AOTO_DEVICE float block_max_f32(float v, float* scratch) {
  v = wave_max(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  float r = scratch[0];
  for (int w = 1; w < kGenThreads / 64; ++w) r = fmaxf(r, scratch[w]);
  __syncthreads();
  return r;
}

AOTO_DEVICE long long block_sum_i64(long long v, long long* scratch) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  long long r = 0;
  for (int w = 0; w < kGenThreads / 64; ++w) r += scratch[w];
  __syncthreads();
  return r;
}

template <bool IS_MAX>
AOTO_DEVICE long long block_extreme_i64(long long v, long long* scratch) {
  for (int o = 32; o > 0; o >>= 1) {
    const long long other = __shfl_xor(v, o, 64);
    v = IS_MAX ? (other > v ? other : v) : (other < v ? other : v);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  long long r = scratch[0];
  for (int w = 1; w < kGenThreads / 64; ++w) r = IS_MAX ? (scratch[w] > r ? scratch[w] : r) : (scratch[w] < r ? scratch[w] : r);
  __syncthreads();
  return r;
}

// (value, index) ordering of argmax / argmin: NaN beats numbers (torch treats
// NaN as the maximum and the minimum), ties go to the lower index, and the
// index kNoIndex stands for "nothing yet".
constexpr long long kNoIndex = 0x7FFFFFFFFFFFFFFFll;

template <bool IS_MAX>
AOTO_DEVICE bool arg_better(float a, long long ia, float b, long long ib) {
  if (ia == kNoIndex) return false;
  if (ib == kNoIndex) return true;
  const bool an = a != a, bn = b != b;
  if (an || bn) return an && (!bn || ia < ib);
  if (a == b) return ia < ib;
  return IS_MAX ? a > b : a < b;
}

template <bool IS_MAX>
AOTO_DEVICE void block_arg_extreme(float& v, long long& idx, float* fscratch, long long* iscratch) {
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const long long oi = __shfl_xor(idx, o, 64);
    if (arg_better<IS_MAX>(ov, oi, v, idx)) {
      v = ov;
      idx = oi;
    }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    fscratch[wave] = v;
    iscratch[wave] = idx;
  }
  __syncthreads();
  v = fscratch[0];
  idx = iscratch[0];
  for (int w = 1; w < kGenThreads / 64; ++w)
    if (arg_better<IS_MAX>(fscratch[w], iscratch[w], v, idx)) {
      v = fscratch[w];
      idx = iscratch[w];
    }
  __syncthreads();
}

// One block per row. Float rows accumulate in f32 (the element type torch and
// MLX use for f32/bf16 reductions), integer rows in int64.
extern "C" __global__ __launch_bounds__(kGenThreads) void aoto_generic_reduce(ReduceArgs a) {
  __shared__ float fscratch[kGenThreads / 64];
  __shared__ long long iscratch[kGenThreads / 64];
  __shared__ long long carry_scratch[kGenThreads];
  for (long long row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const long long base = row * a.in_row_stride;
    const long long obase = row * a.out_row_stride;
    auto at = [&](long long j) { return base + j * a.in_elem_stride; };
    auto out_at = [&](long long j) { return obase + j * a.out_elem_stride; };
    switch (a.op) {
      case AOTO_RED_SUM:
      case AOTO_RED_MEAN: {
        if (a.domain == 1) {
          long long s = 0;
          for (long long j = threadIdx.x; j < a.len; j += kGenThreads) s += load_int(a.in, a.in_dtype, at(j));
          s = block_sum_i64(s, iscratch);
          if (threadIdx.x == 0) store_int(a.out, a.out_dtype, obase, s);
        } else {
          float s = 0.f;
          for (long long j = threadIdx.x; j < a.len; j += kGenThreads) s += (float)load_value(a.in, a.in_dtype, at(j));
          s = block_sum<kGenThreads>(s, fscratch);
          if (a.op == AOTO_RED_MEAN) s = s / (float)a.len;
          if (threadIdx.x == 0) store_float(a.out, a.out_dtype, obase, s);
        }
        break;
      }
      case AOTO_RED_AMAX:
      case AOTO_RED_AMIN: {
        const bool is_max = a.op == AOTO_RED_AMAX;
        if (a.domain == 1) {
          long long m = is_max ? (long long)0x8000000000000000ull : 0x7FFFFFFFFFFFFFFFll;
          for (long long j = threadIdx.x; j < a.len; j += kGenThreads) {
            const long long v = load_int(a.in, a.in_dtype, at(j));
            m = is_max ? (v > m ? v : m) : (v < m ? v : m);
          }
          m = is_max ? block_extreme_i64<true>(m, iscratch) : block_extreme_i64<false>(m, iscratch);
          if (threadIdx.x == 0) store_int(a.out, a.out_dtype, obase, m);
        } else {
          float m = is_max ? -INFINITY : INFINITY;
          bool nan = false;
          for (long long j = threadIdx.x; j < a.len; j += kGenThreads) {
            const float v = (float)load_value(a.in, a.in_dtype, at(j));
            nan |= v != v;
            m = is_max ? fmaxf(m, v) : fminf(m, v);
          }
          const float flag = block_max_f32(nan ? 1.f : 0.f, fscratch);
          m = is_max ? block_max_f32(m, fscratch) : -block_max_f32(-m, fscratch);
          if (threadIdx.x == 0) store_float(a.out, a.out_dtype, obase, flag > 0.f ? NAN : m);
        }
        break;
      }
      case AOTO_RED_ANY:
      case AOTO_RED_ALL: {
        long long hit = 0;
        for (long long j = threadIdx.x; j < a.len; j += kGenThreads) {
          const bool nz = load_value(a.in, a.in_dtype, at(j)) != 0.0;
          hit += (a.op == AOTO_RED_ANY) ? nz : !nz;
        }
        hit = block_sum_i64(hit, iscratch);
        if (threadIdx.x == 0) store_int(a.out, a.out_dtype, obase, a.op == AOTO_RED_ANY ? hit > 0 : hit == 0);
        break;
      }
      case AOTO_RED_ARGMAX:
      case AOTO_RED_ARGMIN: {
        const bool is_max = a.op == AOTO_RED_ARGMAX;
        float v = 0.f;
        long long idx = kNoIndex;
        for (long long j = threadIdx.x; j < a.len; j += kGenThreads) {
          const float x = (float)load_value(a.in, a.in_dtype, at(j));
          const bool take = is_max ? arg_better<true>(x, j, v, idx) : arg_better<false>(x, j, v, idx);
          if (take) {
            v = x;
            idx = j;
          }
        }
        if (is_max)
          block_arg_extreme<true>(v, idx, fscratch, iscratch);
        else
          block_arg_extreme<false>(v, idx, fscratch, iscratch);
        if (threadIdx.x == 0) store_int(a.out, a.out_dtype, obase, idx == kNoIndex ? 0 : idx);
        break;
      }
      case AOTO_RED_SOFTMAX:
      case AOTO_RED_LOG_SOFTMAX: {
        float m = -INFINITY;
        for (long long j = threadIdx.x; j < a.len; j += kGenThreads)
          m = fmaxf(m, (float)load_value(a.in, a.in_dtype, at(j)));
        m = block_max_f32(m, fscratch);
        float s = 0.f;
        for (long long j = threadIdx.x; j < a.len; j += kGenThreads)
          s += expf((float)load_value(a.in, a.in_dtype, at(j)) - m);
        s = block_sum<kGenThreads>(s, fscratch);
        const float ls = logf(s);
        for (long long j = threadIdx.x; j < a.len; j += kGenThreads) {
          const float x = (float)load_value(a.in, a.in_dtype, at(j)) - m;
          store_float(a.out, a.out_dtype, out_at(j), a.op == AOTO_RED_SOFTMAX ? expf(x) / s : x - ls);
        }
        break;
      }
      case AOTO_RED_CUMSUM: {
        // Each thread scans a contiguous chunk; chunk totals are scanned in LDS.
        const long long chunk = (a.len + kGenThreads - 1) / kGenThreads;
        const long long j0 = threadIdx.x * chunk;
        const long long j1 = j0 + chunk < a.len ? j0 + chunk : a.len;
        if (a.domain == 1) {
          long long s = 0;
          for (long long j = j0; j < j1; ++j) s += load_int(a.in, a.in_dtype, at(j));
          carry_scratch[threadIdx.x] = s;
          __syncthreads();
          long long carry = 0;
          for (int t = 0; t < (int)threadIdx.x; ++t) carry += carry_scratch[t];
          for (long long j = j0; j < j1; ++j) {
            carry += load_int(a.in, a.in_dtype, at(j));
            store_int(a.out, a.out_dtype, out_at(j), carry);
          }
        } else {
          float s = 0.f;
          for (long long j = j0; j < j1; ++j) s += (float)load_value(a.in, a.in_dtype, at(j));
          reinterpret_cast<float*>(carry_scratch)[threadIdx.x] = s;
          __syncthreads();
          float carry = 0.f;
          for (int t = 0; t < (int)threadIdx.x; ++t) carry += reinterpret_cast<float*>(carry_scratch)[t];
          for (long long j = j0; j < j1; ++j) {
            carry += (float)load_value(a.in, a.in_dtype, at(j));
            store_float(a.out, a.out_dtype, out_at(j), carry);
          }
        }
        __syncthreads();
        break;
      }
      default:
        break;
    }
  }
}

// Batched strided GEMM: 64x64 output tile per block, k-steps of 16 staged in
// LDS as f32, 4x4 outputs per thread, f32 FMA accumulation.
extern "C" __global__ __launch_bounds__(kGenThreads) void aoto_generic_gemm(GemmArgs g) {
  __shared__ float as[16][64 + 4];
  __shared__ float bs[16][64 + 4];
  const long long batch = blockIdx.z;
  const long long m0 = (long long)blockIdx.y * 64, n0 = (long long)blockIdx.x * 64;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  float acc[4][4] = {};
  for (long long k0 = 0; k0 < g.k; k0 += 16) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int e = threadIdx.x + t * kGenThreads;  // 0..1023
      // A tile: 64 rows x 16 k (element e -> row e / 16, k e % 16)
      const int ar = e >> 4, ak = e & 15;
      const long long gm = m0 + ar, gk = k0 + ak;
      float av = 0.f;
      if (gm < g.m && gk < g.k)
        av = (float)load_value(g.a, g.a_dtype, batch * g.sa_b + gm * g.sa_m + gk * g.sa_k);
      as[ak][ar] = av;
      // B tile: 16 k x 64 cols (element e -> k e / 64, col e % 64)
      const int bk = e >> 6, bn = e & 63;
      const long long gk2 = k0 + bk, gn = n0 + bn;
      float bv = 0.f;
      if (gk2 < g.k && gn < g.n)
        bv = (float)load_value(g.b, g.b_dtype, batch * g.sb_b + gk2 * g.sb_k + gn * g.sb_n);
      bs[bk][bn] = bv;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = as[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const long long gm = m0 + ty * 4 + i;
    if (gm >= g.m) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long long gn = n0 + tx * 4 + j;
      if (gn >= g.n) continue;
      float v = acc[i][j];
      if (g.alpha != 1.f) v *= g.alpha;
      if (g.bias) {
        const float b = (float)load_value(g.bias, g.bias_dtype, batch * g.sbias_b + gm * g.sbias_m + gn * g.sbias_n);
        v = g.beta == 1.f ? v + b : v + g.beta * b;
      }
      store_float(g.c, g.c_dtype, batch * g.sc_b + gm * g.sc_m + gn * g.sc_n, v);
    }
  }
}

// Advanced indexing over the leading dims of a contiguous source; an index out
// of [-size, size) sets *error and writes zeros.
extern "C" __global__ __launch_bounds__(kGenThreads) void aoto_generic_index(IndexArgs a) {
  const long long stride = (long long)gridDim.x * kGenThreads;
  for (long long i = (long long)blockIdx.x * kGenThreads + threadIdx.x; i < a.total; i += stride) {
    const long long r = i % a.inner;
    long long rem = i / a.inner;
    long long ioff[4] = {0, 0, 0, 0};
    for (int d = a.bdims - 1; d >= 0; --d) {
      const long long c = rem % a.bshape[d];
      rem /= a.bshape[d];
      for (int j = 0; j < 4; ++j) ioff[j] += c * a.idx_strides[j][d];
    }
    long long src_off = r;
    bool ok = true;
    for (int j = 0; j < a.nidx; ++j) {
      long long v = load_int(a.idx[j], a.idx_dtype[j], ioff[j]);
      if (v < 0) v += a.dim_size[j];
      if (v < 0 || v >= a.dim_size[j]) {
        ok = false;
        v = 0;
      }
      src_off += v * a.src_stride[j];
    }
    if (!ok && a.error) atomicOr(a.error, 1);
    store_double(a.out, a.dtype, i, ok ? load_value(a.src, a.dtype, src_off) : 0.0);
  }
}

extern "C" __global__ __launch_bounds__(kGenThreads) void aoto_generic_copy(CopyArgs a) {
  const long long stride = (long long)gridDim.x * kGenThreads;
  for (long long i = (long long)blockIdx.x * kGenThreads + threadIdx.x; i < a.total; i += stride) {
    long long rem = i, so = 0, dof = 0;
    for (int d = a.ndim - 1; d >= 0; --d) {
      const long long c = rem % a.shape[d];
      rem /= a.shape[d];
      so += c * a.src_strides[d];
      dof += c * a.dst_strides[d];
    }
    store_double(a.dst, a.dst_dtype, dof, load_value(a.src, a.src_dtype, so));
  }
}

extern "C" __global__ __launch_bounds__(kGenThreads) void aoto_generic_fill(FillArgs a) {
  const long long stride = (long long)gridDim.x * kGenThreads;
  for (long long i = (long long)blockIdx.x * kGenThreads + threadIdx.x; i < a.total; i += stride) {
    if (a.integer)
      store_int(a.dst, a.dtype, i, a.start_i + i * a.step_i);
    else
      store_float(a.dst, a.dtype, i, (float)(a.start + (double)i * a.step));
  }
}

// RMSNorm as the HF modules write it (modeling_llama / modeling_qwen2 RMSNorm):
// x32 = float(x); r = rsqrt(mean(x32^2) + eps); y = w * cast_mid(x32 * r).
extern "C" __global__ __launch_bounds__(kGenThreads) void aoto_generic_rms_norm(RmsArgs a) {
  __shared__ float scratch[kGenThreads / 64];
  for (long long row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const long long base = row * a.hidden;
    float ss = 0.f;
    for (long long j = threadIdx.x; j < a.hidden; j += kGenThreads) {
      const float v = (float)load_value(a.x, a.x_dtype, base + j);
      ss += v * v;
    }
    ss = block_sum<kGenThreads>(ss, scratch);
    const float r = 1.0f / sqrtf(ss / (float)a.hidden + a.eps);
    for (long long j = threadIdx.x; j < a.hidden; j += kGenThreads) {
      float y = (float)load_value(a.x, a.x_dtype, base + j) * r;
      if (a.mid_dtype == AOTO_DT_BF16) y = round_bf16(y);
      if (a.has_weight) y = (float)load_value(a.w, a.w_dtype, j) * y;
      store_float(a.out, a.out_dtype, base + j, y);
    }
  }
}

// Scaled dot-product attention, one (batch, head, query row) per block:
// scores into LDS, f32 softmax, then each thread owns output columns. A bool
// mask keeps True entries, a float mask is added; is_causal keeps j <= i
// (aligned to the top-left, as torch's is_causal). A row with every key
// masked produces zeros (the reference's safe softmax).
constexpr int kAttnMaxKeys = 8192;

extern "C" __global__ __launch_bounds__(kGenThreads) void aoto_generic_attention(AttnArgs a) {
  __shared__ float p[kAttnMaxKeys];
  __shared__ float scratch[kGenThreads / 64];
  const int row = blockIdx.x;  // query index
  const int h = blockIdx.y % a.heads;
  const int b = blockIdx.y / a.heads;
  const int kvh = h / (a.heads / a.kv_heads);
  const long long qb = b * a.qs[0] + h * a.qs[1] + row * a.qs[2];
  float m = -INFINITY;
  for (int j = threadIdx.x; j < a.lk; j += kGenThreads) {
    float s = -INFINITY;
    bool keep = !(a.causal && j > row);
    float add = 0.f;
    if (a.mask) {
      const long long mo = b * a.ms[0] + h * a.ms[1] + row * a.ms[2] + j * a.ms[3];
      if (a.mask_dtype == AOTO_DT_BOOL)
        keep = keep && static_cast<const uint8_t*>(a.mask)[mo] != 0;
      else
        add = (float)load_value(a.mask, a.mask_dtype, mo);
    }
    if (keep) {
      const long long kb = b * a.ks[0] + kvh * a.ks[1] + j * a.ks[2];
      float dot = 0.f;
      for (int d = 0; d < a.d; ++d)
        dot = fmaf((float)load_value(a.q, a.q_dtype, qb + d * a.qs[3]),
                   (float)load_value(a.k, a.k_dtype, kb + d * a.ks[3]), dot);
      s = dot * a.scale + add;
    }
    p[j] = s;
    m = fmaxf(m, s);
  }
  m = block_max_f32(m, scratch);
  float l = 0.f;
  for (int j = threadIdx.x; j < a.lk; j += kGenThreads) {
    const float e = (m == -INFINITY) ? 0.f : expf(p[j] - m);
    p[j] = e;
    l += e;
  }
  l = block_sum<kGenThreads>(l, scratch);  // ends with a barrier: p is complete
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  const long long ob = ((long long)(b * a.heads + h) * a.lq + row) * a.dv;
  for (int d = threadIdx.x; d < a.dv; d += kGenThreads) {
    float acc = 0.f;
    for (int j = 0; j < a.lk; ++j) {
      if (p[j] == 0.f) continue;
      acc = fmaf(p[j], (float)load_value(a.v, a.v_dtype, b * a.vs[0] + kvh * a.vs[1] + j * a.vs[2] + d * a.vs[3]),
                 acc);
    }
    store_float(a.out, a.out_dtype, ob + d, acc * inv);
  }
}

}  // namespace aoto
