// Kernel-argument records of the generic graph kernels (generic.h), shared by
// the device code and the host launchers: plain structs passed by value as one
// kernel argument each. Strides and shapes are in elements, up to 8 dims.
#pragma once

#include <stdint.h>

namespace aoto {

constexpr int kMaxDims = 8;

// One elementwise operand: a strided view broadcast to the output shape
// (stride 0 along broadcast dims), or a scalar when data == nullptr.
struct Operand {
  const void* data;
  int dtype;
  int pad;
  long long strides[kMaxDims];
  double value;
};

struct EwArgs {
  int op;
  int domain;  // compute domain: 0 f32, 1 int64, 2 compare in f64, 3 select
  int ndim;
  int out_dtype;
  long long total;
  long long shape[kMaxDims];
  void* out;  // contiguous output
  double alpha;
  Operand in[3];
};

// Row reduction / scan over a [rows, len] view.
struct ReduceArgs {
  int op;
  int domain;  // 0 f32, 1 int64
  int in_dtype;
  int out_dtype;
  long long rows;
  long long len;
  const void* in;
  long long in_row_stride;
  long long in_elem_stride;
  void* out;
  long long out_row_stride;
  long long out_elem_stride;
};

// C[b][m][n] = alpha * sum_k A[b][m][k] B[b][k][n] + beta * bias (broadcast), f32 accumulation.
struct GemmArgs {
  const void* a;
  const void* b;
  const void* bias;
  void* c;
  int a_dtype, b_dtype, bias_dtype, c_dtype;
  long long batch, m, n, k;
  long long sa_b, sa_m, sa_k;
  long long sb_b, sb_k, sb_n;
  long long sbias_b, sbias_m, sbias_n;
  long long sc_b, sc_m, sc_n;
  float alpha, beta;
};

// out[bcoord..., r] = src[sum_j idx_j[bcoord] * src_stride_j + r]: advanced
// indexing over the leading dims of a contiguous source.
struct IndexArgs {
  const void* src;
  int dtype;
  int nidx;
  int bdims;
  int pad;
  long long bshape[kMaxDims];
  const void* idx[4];
  int idx_dtype[4];
  long long idx_strides[4][kMaxDims];
  long long dim_size[4];
  long long src_stride[4];
  long long inner;
  long long total;
  void* out;
  int* error;
};

// Strided copy with element-type conversion.
struct CopyArgs {
  const void* src;
  void* dst;
  int src_dtype;
  int dst_dtype;
  int ndim;
  int pad;
  long long total;
  long long shape[kMaxDims];
  long long src_strides[kMaxDims];
  long long dst_strides[kMaxDims];
};

// Fill (step == 0) or arange: dst[i] = start + i * step, contiguous.
struct FillArgs {
  void* dst;
  int dtype;
  int integer;  // 1: compute in int64 (start_i, step_i)
  long long total;
  double start, step;
  long long start_i, step_i;
};

// HF-style RMSNorm over rows of a contiguous [rows, hidden] input:
//   y = w * cast_mid(x32 * rsqrt(mean(x32^2) + eps))
struct RmsArgs {
  const void* x;
  const void* w;
  void* out;
  int x_dtype, w_dtype, mid_dtype, out_dtype;
  long long rows, hidden;
  float eps;
  int has_weight;
};

// Scaled dot-product attention, one query row per block.
struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* mask;
  void* out;
  int q_dtype, k_dtype, v_dtype, mask_dtype, out_dtype;
  int causal;
  int batch, heads, kv_heads, lq, lk, d, dv;
  long long qs[4], ks[4], vs[4], ms[4];  // (b, h, l, d) strides; mask (b, h, lq, lk)
  float scale;
};

}  // namespace aoto
