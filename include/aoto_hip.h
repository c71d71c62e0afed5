/*
 * aoto_hip.h - C ABI of the gfx950 kernel backend for aotolith's W4 decoder path.
 *
 * Every entry point takes raw device pointers, static shape/attribute values and
 * a HIP stream (passed as void*, i.e. hipStream_t), enqueues work on that stream
 * and returns a status (AOTO_OK == 0). On failure,
 * aoto_hip_last_error() returns the calling thread's message. The library never
 * allocates or frees caller memory and keeps no per-call state; the kernels come
 * from a gfx950 code object installed with aoto_hip_load_code_object() (one
 * module per device, guarded by a mutex).
 *
 * bf16 tensors are passed as void* to 16-bit storage; int4 weights are the
 * reference's packed format: int32 words [N, K/8] (code 8j+k of a row at bits 4k
 * of word j, two's complement) with bf16 group scales [N, K/group].
 *
 * Each declaration cites the reference (aotolith 0.68.0, src/aotolith/...)
 * interface it replaces: there, every kernel is an MSL source string emitted per
 * graph node and launched through mx.fast.metal_kernel.
 */
#ifndef AOTO_HIP_H
#define AOTO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AOTO_OK 0
#define AOTO_ERR_ARGUMENT 1       /* malformed arguments (null pointer, bad size) */
#define AOTO_ERR_NO_CODE_OBJECT 2 /* no code object installed on the current device */
#define AOTO_ERR_HIP 3            /* a HIP runtime call failed */
#define AOTO_ERR_UNSUPPORTED 4    /* shape outside this kernel's limits: select another impl */

#define AOTO_HIP_ABI_VERSION 1

/* ABI version of the loaded library (AOTO_HIP_ABI_VERSION at build time). */
int aoto_hip_abi_version(void);

/* Copy the calling thread's last error message into buf (NUL-terminated,
 * truncated to size). Returns the full message length. */
size_t aoto_hip_last_error(char* buf, size_t size);

/* Install a gfx950 code object (the bytes of an .hsaco) as the kernel module of
 * the current device, replacing any previous one. Replaces the reference's
 * kernel shell and cache (codegen/msl.py:625-646) and, on artifact reload, its
 * re-emission of MSL (artifact.py:367-384): the stored code object is loaded
 * as-is instead of regenerating source. */
int aoto_hip_load_code_object(const void* image, size_t size);

/* Unload the current device's module. */
int aoto_hip_unload_code_object(void);

/* 1 when a module is installed on the current device, else 0. */
int aoto_hip_code_object_loaded(void);

/* Symmetric int4 group quantizer + packer, bit-exact with quantize.py:95-152 and
 * the bf16 scale cast of models/quantized.py:133-163 (pack_weight).
 * weight: [rows, inner] bf16 (weight_is_f32 == 0) or f32; group % 8 == 0 and
 * divides inner. Writes packed int32 [rows, inner/8], scales bf16
 * [rows, inner/group] and, when scales_f32 is non-null, the f32 scales. */
int aoto_hip_w4_quantize(const void* weight, int weight_is_f32, int rows, int inner, int group,
                         int32_t* packed, void* scales_bf16, float* scales_f32, void* stream);

/* bf16(code * scale): the dequantize_i4 op in the scales' dtype
 * (models/quantized.py:61-82; Metal dequant kernel codegen/quantize.py:27-153).
 * out: bf16 [rows, inner]. */
int aoto_hip_w4_dequantize(const int32_t* packed, const void* scales, int rows, int inner,
                           int group, void* out, void* stream);

/* Decode GEMV over a packed W4 weight, one activation row (M == 1). Replaces the
 * packed GEMV emitter _emit_quantized_gemv_matmul_source (codegen/matmul.py:542-739)
 * with its epilogues (:571-602) and RMSNorm prologue (codegen/norm.py:45-72):
 *   x          bf16 [K]
 *   words      int32 [N, K/8], scales bf16 [N, K/group]   (gate rows when paired)
 *   up_words, up_scales   second projection for the paired silu_mul epilogue
 *                         (passes/fusion.py:215-403), or NULL
 *   norm_weight bf16 [K] for the fused RMSNorm prologue, or NULL; eps its epsilon
 *   bias        bf16 [N] addmm operand (q/k/v bias or residual), or NULL
 *   y           bf16 [N]
 * Limits: K % 32 == 0, group % 32 == 0, group divides K, K <= 32768, N >= 1.
 * lanes_per_row: 4, 8, 16, 32 or 64 lanes per output row, 0 for the default. */
int aoto_hip_w4_gemv(const void* x, const int32_t* words, const void* scales,
                     const int32_t* up_words, const void* up_scales, const void* norm_weight,
                     float eps, const void* bias, float alpha, float beta, void* y, int K, int N,
                     int group, int lanes_per_row, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AOTO_HIP_H */
