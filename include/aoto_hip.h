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
 * of word j, two's complement) with bf16 group scales [N, K/group]. int8
 * weights (the aoto_hip_w8_* entry points) are int32 words [N, K/4], code 4j+k
 * at bits 8k of word j, with the same bf16 group scales.
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

#define AOTO_HIP_ABI_VERSION 19

/* ABI version of the loaded library (AOTO_HIP_ABI_VERSION at build time). */
int aoto_hip_abi_version(void);

/* Record the kernel symbols this host thread launches (the counterpart of the
 * reference's KernelSelection.artifact_name, selection.py:19-34, which names the
 * kernel each node emitted): enable != 0 starts recording (clearing the record),
 * 0 stops. Returns the previous state. */
int aoto_hip_trace_launches(int enable);

/* Copy the recorded symbols, newline-separated, into buf (NUL-terminated) and
 * clear the record when they fit; returns the record's length in bytes (call with
 * size 0 to size the buffer). */
size_t aoto_hip_take_launches(char* buf, size_t size);

/* Copy the calling thread's last error message into buf (NUL-terminated,
 * truncated to size). Returns the full message length. */
size_t aoto_hip_last_error(char* buf, size_t size);

/* Install a gfx950 code object (the bytes of an .hsaco) as the kernel module of
 * the current device: later launches use its kernels. The module it replaces is
 * unloaded at once when no captured graph is held (aoto_hip_hold_graphs), else
 * kept until the last hold is released, because those graphs launch its kernels
 * by handle. Replaces the reference's kernel shell and cache
 * (codegen/msl.py:625-646) and, on artifact reload, its re-emission of MSL
 * (artifact.py:367-384): the stored code object is loaded as-is instead of
 * regenerating source. */
int aoto_hip_load_code_object(const void* image, size_t size);

/* No counterpart in the reference (its runtime has no captured graphs). Count
 * (+1) or release (-1) a captured HIP graph whose nodes launch kernels of the
 * loaded code objects; process-wide. A release that brings the count to zero
 * unloads the modules replaced in the meantime. A count below zero is refused. */
int aoto_hip_hold_graphs(int delta);
/* The current number of held graphs. */
int aoto_hip_graph_holds(void);

/* Unload the current device's module and every module it replaced. Refused
 * (AOTO_ERR_ARGUMENT) while any captured graph is held: replaying one afterwards
 * would execute unloaded code. */
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

/* Prefill W4 GEMM, Y[M, N] = X[M, K] . bf16(code * scale)[N, K]^T with at most
 * one fused epilogue. Replaces the prefill pair the reference runs for M > 1:
 * the dequant kernel (codegen/quantize.py:27-153) feeding the tiled GEMM
 * _emit_mpp_matmul_source (codegen/matmul.py:1228-1473) with its bias /
 * residual / silu_mul epilogue (:1443-1471, 1721-1742; passes/fusion.py:406-498):
 *   bias     bf16 [N]     -> bf16(bias[n] + acc)        (packed q/k/v bias)
 *   residual bf16 [M, N]  -> bf16(residual[m][n] + acc)
 *   gate     bf16 [M, N]  -> bf16(acc * silu(gate[m][n]))
 * Limits: K % 64 == 0, N % 16 == 0, group % 32 == 0 dividing K. x 16-byte and
 * y/bias/residual/gate 8-byte aligned. tile: 0 chooses; 12/14/18/24/28 the
 * 16x16x32-MFMA kernel (n tiles x m tiles of 16 per wave; 12: 32-row blocks);
 * 241/242/243/281/441 the wide-tile 32x32x16 kernel for long prompts (100 *
 * waves per block / 2 + 10 * 32-row tiles per wave + 32-column tiles per wave;
 * needs K % 128 == 0 and an even number of power-of-two groups per row; 8-bit
 * codes: 241, 242, 441; the paired gate/up: 241); 822 / 823 (the paired gate/up: 821, and for
 * short prompts 812 / 811) the dequant-once kernel (each packed tile expanded once per block into
 * LDS; 256 x 128 / 256 x 192 / 256 x (64 + 64) blocks of 8 waves, 128 x (64 + 64) / 128 x (32 +
 * 32) blocks of 4 waves; 4-bit codes, unsplit, no gate epilogue, K % 64 == 0, an even number of
 * power-of-two groups per row, x and the packed words under 2 GiB); 814 / 813 its split-K form
 * for single projections (128 x 64 / 128 x 32 blocks of 4 waves storing f32 partials that the
 * reduce launch sums with the epilogue, at every split count, so they always take a workspace).
 * Automatic codes take the dequant-once kernel for 4-bit codes from M >= 1024 when its grid's
 * last round of 256 blocks is at least 90% full, for a paired gate/up of 32-256 rows on 128-row
 * blocks (812 where that gives >= 128 blocks from 65 rows, else 811 within 256 blocks), for a
 * single projection of 32-256 rows with K >= 2048 and no RoPE epilogue the split form (814
 * where that gives >= 64 column blocks, else 813), else the wide kernel from M >= 512 when
 * K % 256 == 0 (group <= 128), else the 16x16 kernel. splits: 0 chooses (small
 * grids split the reduction), else the split-K count; a split launch stores f32
 * partial tiles in `workspace` (aoto_hip_w4_gemm_workspace() bytes, 16-byte
 * aligned) and a second launch sums them and applies the epilogue. Every plan is
 * a fixed function of the arguments, so results are reproducible across calls and
 * processes. y must not alias x. */
int aoto_hip_w4_gemm(const void* x, const int32_t* words, const void* scales, const void* bias,
                     const void* residual, const void* gate, void* y, int M, int N, int K, int group,
                     int tile, int splits, void* workspace, void* stream);

/* Bytes of workspace aoto_hip_w4_gemm needs for these arguments: the split-K
 * partials (0 when it does not split). */
size_t aoto_hip_w4_gemm_workspace(int M, int N, int K, int tile, int splits);

/* No counterpart in the reference. aoto_hip_w4_gemm for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the same arguments and results without the
 * workspace. A split-K plan keeps its f32 partials in a static device buffer of
 * AOTO_HIP_NOALLOC_SCRATCH_BYTES that the library holds on each GPU until the
 * process ends. With automatic codes (tile = splits = 0) the split count of the
 * automatic plan is lowered, to one at least, until the partials fit; explicit codes
 * whose plan needs more (aoto_hip_w4_gemm_workspace() bytes) are refused with
 * AOTO_ERR_UNSUPPORTED.
 * Nothing is allocated or freed. All calls on one GPU share its buffer: calls that
 * overlap in time on one device (different streams) race. */
#define AOTO_HIP_NOALLOC_SCRATCH_BYTES (16u << 20)
int aoto_hip_w4_gemm_noalloc(const void* x, const int32_t* words, const void* scales, const void* bias,
                             const void* residual, const void* gate, void* y, int M, int N, int K, int group,
                             int tile, int splits, void* stream);

/* Symmetric int8 group quantizer + packer, bit-exact with quantize.py:155-172
 * (quantize_int8: scale = max|w| / 127, an all-zero group 1/127, codes
 * clip(rint(w / scale), -128, 127)) and the bf16 scale cast of
 * models/quantized.py:133-172 (pack_weight_int8). Arguments as
 * aoto_hip_w4_quantize; group % 4 == 0. packed: int32 [rows, inner/4]. */
int aoto_hip_w8_quantize(const void* weight, int weight_is_f32, int rows, int inner, int group,
                         int32_t* packed, void* scales_bf16, float* scales_f32, void* stream);

/* bf16(code * scale) of an int8 pack: the dequantize_i8 op in the scales'
 * dtype (models/quantized.py:84-107; Metal kernel codegen/quantize.py:66-99,
 * 155-190). out: bf16 [rows, inner], 8-byte aligned. */
int aoto_hip_w8_dequantize(const int32_t* packed, const void* scales, int rows, int inner,
                           int group, void* out, void* stream);

/* Decode GEMV over a packed int8 weight, one activation row (M == 1): the
 * eight-bit emitter _emit_quantized_gemv_int8_source (codegen/matmul.py:742-929)
 * with the same prologue and epilogues as aoto_hip_w4_gemv (words are int32
 * [N, K/4]). Limits: K % 16 == 0, group % 16 == 0 dividing K, K <= 32768. */
int aoto_hip_w8_gemv(const void* x, const int32_t* words, const void* scales,
                     const int32_t* up_words, const void* up_scales, const void* norm_weight,
                     float eps, const void* bias, float alpha, float beta, void* y, int K, int N,
                     int group, void* stream);

/* Prefill GEMM over a packed int8 weight: aoto_hip_w4_gemm with words int32
 * [N, K/4] (8-byte aligned); the reference's prefill pair for eight bits is
 * dequantize_i8 (codegen/quantize.py:155-190) feeding the same tiled GEMM.
 * Same limits, tile codes, split-K and workspace (aoto_hip_w4_gemm_workspace()
 * bytes: the plan does not depend on the code width). */
int aoto_hip_w8_gemm(const void* x, const int32_t* words, const void* scales, const void* bias,
                     const void* residual, const void* gate, void* y, int M, int N, int K, int group,
                     int tile, int splits, void* workspace, void* stream);

/* The prefill MLP's gate and up projections in one pass: y[M, N] =
 * bf16(up . x * silu(bf16(gate . x))) - the reference's gate GEMM followed by
 * the up GEMM with the silu_mul epilogue (codegen/matmul.py:1443-1471,
 * 1721-1742; passes/fusion.py:406-498), with X read once. gate/up words and
 * scales as aoto_hip_w4_gemm (int4) / aoto_hip_w8_gemm (int8), both [N, K].
 * Limits, tile and splits as aoto_hip_w4_gemm; a split launch needs
 * aoto_hip_w4_gemm_gate_up_workspace() bytes (gate and up partials), as does
 * the long-prefill path (both unpacked weights, the up projection's f32 product
 * and the bf16 gate). */
int aoto_hip_w4_gemm_gate_up(const void* x, const int32_t* gate_words, const void* gate_scales,
                             const int32_t* up_words, const void* up_scales, void* y, int M, int N, int K,
                             int group, int tile, int splits, void* workspace, void* stream);
int aoto_hip_w8_gemm_gate_up(const void* x, const int32_t* gate_words, const void* gate_scales,
                             const int32_t* up_words, const void* up_scales, void* y, int M, int N, int K,
                             int group, int tile, int splits, void* workspace, void* stream);

/* A decoder layer's o or down projection followed by the next block's RMSNorm
 * (models/decoder.py:150-204 layer order; codegen/matmul.py:1721-1742 residual
 * epilogue; the norm as aoto_hip_rms_norm): y[M, N] = bf16(x . W^T + residual),
 * then norm_out = bf16((y * rsqrt(mean(y^2) + eps)) * norm_weight) per row.
 * y equals aoto_hip_w4_gemm with the residual epilogue bit for bit; a split
 * plan sums the partials and normalizes in one launch, its sum of squares a
 * block sum (norm_out within one bf16 rounding of aoto_hip_rms_norm's). y may alias the residual; norm_out may alias neither. Limits,
 * tile, splits and workspace as aoto_hip_w4_gemm, plus N % 8 == 0, N <= 4096
 * and 16-byte aligned y, residual, norm_weight and norm_out. */
int aoto_hip_w4_gemm_residual_norm(const void* x, const int32_t* words, const void* scales, const void* residual,
                                   void* y, int M, int N, int K, int group, int tile, int splits, void* workspace,
                                   const void* norm_weight, float eps, void* norm_out, void* stream);
int aoto_hip_w8_gemm_residual_norm(const void* x, const int32_t* words, const void* scales, const void* residual,
                                   void* y, int M, int N, int K, int group, int tile, int splits, void* workspace,
                                   const void* norm_weight, float eps, void* norm_out, void* stream);

/* The prefill's packed q/k/v projection with its RoPE and the layer's cache fill:
 * the reference's q/k/v matmul with the bias epilogue (codegen/matmul.py:1228-1473,
 * 1443-1471) followed by RoPE of q and k (codegen/index.py:22-126, tables of
 * models/decoder.py:323-334) and the prefill module's returned key/value window
 * (models/decoder.py:524-561, 870-887) - the values of aoto_hip_w4_gemm (bias) then
 * aoto_hip_rope_qkv_prefill (batch 1), in one launch: unsplit, when a block's
 * columns are whole heads, RoPE and the cache fill run in the GEMM's epilogue;
 * split, the split sum, bias, RoPE and cache fill share the second launch.
 * x [M, K]; the weight packs N = (Hq + 2 Hkv) * head_dim rows; y [M, N] receives
 * the projection; q_out [Hq, M, head_dim]; pair [2, Hkv, capacity, head_dim] gets
 * rotated keys / values at slots slot0 .. slot0 + M - 1 (slots below slot0 zeroed
 * when zero_prefix != 0); positions[M] int64. tile and splits as aoto_hip_w4_gemm,
 * with 0 / 0 choosing, below the wide kernel's rows, the unsplit epilogue form
 * whenever it applies (32-row blocks up to 128 rows), and from them the wide kernel
 * with the RoPE / cache fill kernel after it;
 * workspace: aoto_hip_w4_gemm_qkv_rope_workspace() bytes. */
int aoto_hip_w4_gemm_qkv_rope(const void* x, const int32_t* words, const void* scales, const void* bias, void* y,
                              int M, int K, int group, int tile, int splits, void* workspace, const int64_t* positions,
                              const void* cos_table, const void* sin_table, void* q_out, void* pair, int query_heads,
                              int kv_heads, int head_dim, int capacity, int slot0, int zero_prefix, void* stream);
int aoto_hip_w8_gemm_qkv_rope(const void* x, const int32_t* words, const void* scales, const void* bias, void* y,
                              int M, int K, int group, int tile, int splits, void* workspace, const int64_t* positions,
                              const void* cos_table, const void* sin_table, void* q_out, void* pair, int query_heads,
                              int kv_heads, int head_dim, int capacity, int slot0, int zero_prefix, void* stream);
/* Workspace bytes of aoto_hip_w{4,8}_gemm_qkv_rope with these arguments (0: the
 * fused plan does not split K). */
size_t aoto_hip_w4_gemm_qkv_rope_workspace(int M, int K, int tile, int splits, int query_heads, int kv_heads,
                                           int head_dim);

/* Bytes of workspace the gate/up entry points need (0 when the fused plan does
 * not split). */
size_t aoto_hip_w4_gemm_gate_up_workspace(int M, int N, int K, int tile, int splits);

/* Row RMSNorm, out = bf16((x * rsqrt(mean(x^2) + eps)) * weight) over [rows, hidden]
 * (codegen/norm.py:75-323, _compile_normalization(kind="rms_norm");
 * runtime/mlx_ops/normalization.py:73-119). hidden % 8 == 0. */
int aoto_hip_rms_norm(const void* x, const void* weight, float eps, void* out, int rows, int hidden,
                      void* stream);

/* RoPE over [rows, head_dim] rows (codegen/index.py:22-126, _compile_rope;
 * runtime/mlx_ops/__init__.py:276-280): row r uses the table row
 * positions[(r / rows_per_position) % position_count]; out = bf16(x * cos +
 * rotate_half(x) * sin). Tables are the [capacity, head_dim] bf16 cos/sin of
 * models/decoder.py:323-334. */
int aoto_hip_rope(const void* x, const void* cos_table, const void* sin_table, const int64_t* positions,
                  int rows_per_position, int position_count, void* out, int64_t rows, int head_dim,
                  void* stream);

/* Prefill RoPE fused with the cache fill for one layer: from the packed q/k/v
 * projection qkv [batch, tokens, (Hq + 2 Hkv) * head_dim], writes rotated
 * queries q_out [batch, Hq, tokens, head_dim] and the layer's key/value window
 * pair [2, batch, Hkv, capacity, head_dim] at slots slot0 .. slot0 + tokens
 * (slots below slot0 zeroed when zero_prefix). Replaces the prefill module's two
 * RoPE launches and the compact-cache stack + pad_cache of
 * models/decoder.py:524-561, 870-887. positions: int64 [batch, tokens]. */
int aoto_hip_rope_qkv_prefill(const void* qkv, const int64_t* positions, const void* cos_table,
                              const void* sin_table, void* q_out, void* pair, int batch, int tokens,
                              int query_heads, int kv_heads, int head_dim, int capacity, int slot0,
                              int zero_prefix, void* stream);

/* Decode RoPE + KV-cache append (rope_kv_cache_append, codegen/kv_cache.py:96-215,
 * 295-383; semantics runtime/mlx_ops/__init__.py:207-236). Rotates the step's q
 * and k out of the projection row [batch, row_width] with the table row at
 * `position`; q_out [batch, Hq, head_dim].
 *   mode 0 (the reference op): pair_out = pair_in shifted down one slot with
 *          (k_rot, v) at capacity - 1; pair_in/pair_out are one layer's
 *          [2, batch, Hkv, capacity, head_dim] windows and must not overlap.
 *   mode 1 (ring): (k_rot, v) written in place at `slot` of pair_out.
 * step_state: NULL, or (ring mode) an int32 device array {position, valid,
 * ring_offset, slot} read by the kernel in place of `position` and `slot`. */
int aoto_hip_rope_kv_cache_append(const void* row, int row_width, const void* cos_table, const void* sin_table,
                                  int position, const void* pair_in, void* pair_out, void* q_out, int batch,
                                  int query_heads, int kv_heads, int capacity, int head_dim, int query_start,
                                  int key_start, int value_start, int mode, int slot,
                                  const int32_t* step_state, void* stream);

/* Bytes of the split-K workspace aoto_hip_decode_attention needs for these
 * shapes and `splits` (0 = the launcher's own choice). */
size_t aoto_hip_decode_attention_workspace(int batch, int query_heads, int kv_heads, int capacity, int head_dim,
                                           int splits);

/* Single-query GQA attention over a key/value window (the decode kernel
 * _emit_decode_attention_source, codegen/attention.py:447-656, 761-815; fallback
 * runtime/mlx_ops/attention.py:89-122). q [batch, Hq, head_dim]; keys/values at
 * base + b * kv_batch_stride + h * kv_head_stride + slot * head_dim (elements);
 * out [batch, Hq, head_dim]. Kept slots: mask[b * mask_batch_stride + slot] != 0
 * when mask is non-null, else the last `valid` logical slots, logical slot =
 * (slot - ring_offset) mod capacity. head_dim 64 or 128; Hq / Hkv in {1,2,4,7,8}.
 * workspace: NULL (one block per kv head, capacity <= 512) or a buffer of
 * aoto_hip_decode_attention_workspace() bytes for the split-K records, which a
 * second launch merges (splits 0 = choose: one block per kv head up to 512
 * keys); calls sharing one workspace must be ordered on one stream.
 * step_state: NULL, or the int32 device array {position, valid, ring_offset,
 * slot} read in place of valid / ring_offset. */
int aoto_hip_decode_attention(const void* q, const void* keys, const void* values, int64_t kv_batch_stride,
                              int64_t kv_head_stride, const uint8_t* mask, int mask_batch_stride, int valid,
                              int ring_offset, int batch, int query_heads, int kv_heads, int capacity,
                              int head_dim, float scale, int splits, void* workspace,
                              const int32_t* step_state, void* out, void* stream);

/* Decode RoPE + KV append + attention in one launch (the ring-buffer decode
 * step): the rope_kv_cache_append node (codegen/kv_cache.py:96-215) folded into
 * the decode attention (codegen/attention.py:447-656). From the projection row
 * [batch, row_width] it rotates the queries and the new key with the table row
 * at `position`, writes (k_rot, v) in place at slot `slot` of keys/values
 * (layout as for aoto_hip_decode_attention) and attends over the window with
 * the new pair included; kept slots as for aoto_hip_decode_attention (valid,
 * ring_offset). out [batch, Hq, head_dim]. step_state as above supplies
 * {position, valid, ring_offset, slot} on the device. rope_rows, when non-null,
 * is the cos row then the sin row (2 * head_dim bf16) of the step's position,
 * used instead of the tables (aoto_hip_argmax_finish keeps it current), so the
 * kernel's loads do not wait for the step state. */
int aoto_hip_decode_rope_attention(const void* row, int row_width, int query_start, int key_start,
                                   int value_start, const void* cos_table, const void* sin_table, void* keys,
                                   void* values, int64_t kv_batch_stride, int64_t kv_head_stride, int position,
                                   int slot, int valid, int ring_offset, int batch, int query_heads, int kv_heads,
                                   int capacity, int head_dim, float scale, int splits, void* workspace,
                                   const int32_t* step_state, const void* rope_rows, void* out, void* stream);

/* Advance a decode loop's device step state {position, valid, ring_offset,
 * slot} by one token (ring offset and slot wrap at capacity). The greedy loop
 * of models/decoder.py:1054-1087 does this on the host between steps; on the
 * device the captured step replays unchanged. */
int aoto_hip_step_advance(int32_t* step_state, int capacity, void* stream);

/* Prefill GQA attention on MFMA (the flash kernels of codegen/attention.py:68-422,
 * 671-759 and 817-1400, with the SDPA legalization's scale and safe_softmax,
 * legalize/attention.py:105-170). q [batch, Hq, tokens, head_dim]; keys/values as
 * for decode with key_tokens rows; out [batch, tokens, Hq * head_dim]. Kept pairs:
 * mask[b * mask_batch_stride + i * key_tokens + j] != 0 when mask is non-null,
 * else j >= key_start and (when causal) j <= i + key_tokens - tokens - the
 * reference's prefill_mask (models/decoder.py:226-247) at key_start =
 * tokens - length. Fully masked query rows give 0. head_dim 64 or 128. */
int aoto_hip_prefill_attention(const void* q, const void* keys, const void* values, int64_t kv_batch_stride,
                               int64_t kv_head_stride, const uint8_t* mask, int64_t mask_batch_stride, int causal,
                               int key_start, int batch, int tokens, int key_tokens, int query_heads,
                               int kv_heads, int head_dim, float scale, void* out, void* stream);

/* Embedding gather out[i] = weight[ids[i]] (the embedding op, runtime/bounds.py:
 * 104-107). ids are int64 in device memory. An id outside [0, vocab) yields a
 * zero row and sets *error = 1 when error is non-null (checked, not faulted). */
int aoto_hip_embedding(const void* weight, const int64_t* ids, int count, int hidden, int64_t vocab, void* out,
                       int* error, void* stream);

/* Greedy argmax per row of bf16 logits, first index on ties (mx.argmax in the
 * greedy loop, models/decoder.py:1069, 1080). out int64 [rows]. With history
 * non-null (rows == 1): history[*history_len] = token, ++*history_len. */
int aoto_hip_argmax(const void* logits, int rows, int n, int64_t row_stride, int64_t* out, int64_t* history,
                    int* history_len, void* stream);

/* LM-head W4 GEMV (the packed GEMV with the final RMSNorm prologue,
 * codegen/matmul.py:542-739 with codegen/norm.py:45-72) fused with the first
 * half of the greedy argmax that follows it (models/decoder.py:1069, 1080):
 * y = the GEMV's bf16 logits [N] as aoto_hip_w4_gemv writes them, plus one
 * argmax key per wave of the launch in keys[0 .. aoto_hip_w4_gemv_argmax_keys)
 * for aoto_hip_argmax_finish. norm_weight may be null (no prologue). */
size_t aoto_hip_w4_gemv_argmax_keys(int K, int N, int group); /* 0: shape unsupported */
int aoto_hip_w4_gemv_argmax(const void* x, const int32_t* words, const void* scales, const void* norm_weight,
                            float eps, void* y, int K, int N, int group, uint64_t* keys, size_t key_count,
                            void* stream);

/* Second half of the fused greedy argmax (mx.argmax, models/decoder.py:1069,
 * 1080, first index on ties) and the loop bookkeeping around it: reduces the
 * keys to *token_out; then, each when its pointer is non-null, appends the
 * token to history (history[*history_len], ++*history_len), advances the decode
 * step state like aoto_hip_step_advance, and gathers the token's embedding row
 * (the next step's embedding take, runtime/bounds.py:104-107) into hidden_out
 * (zeros and *error = 1 if the token is not a row of the table), and with the
 * step state copies the cos/sin rows of the advanced position from the tables
 * ([capacity, head_dim] bf16, head_dim <= 256) into rope_rows (2 * head_dim)
 * for the next step's aoto_hip_decode_rope_attention (kept as is when that
 * position is past the tables). */
int aoto_hip_argmax_finish(const uint64_t* keys, int key_count, int64_t* token_out, int64_t* history,
                           int* history_len, int32_t* step_state, int capacity, const void* embedding,
                           int64_t embedding_rows, int hidden, void* hidden_out, int* error,
                           const void* cos_table, const void* sin_table, int head_dim, void* rope_rows,
                           void* stream);

/* The greedy loop's argmax finish (aoto_hip_argmax_finish) folded into the
 * prologue of the next step's first GEMV, the layer-0 q/k/v projection
 * (models/decoder.py:1054-1087: the argmax, the next step's embedding take,
 * runtime/bounds.py:104-107, and the packed q/k/v GEMV with its RMSNorm
 * prologue and bias, codegen/matmul.py:542-739, codegen/norm.py:45-72). Every
 * block reduces the keys an aoto_hip_w4_gemv_argmax launch wrote to the token
 * and uses that token's embedding row as x; y = the GEMV aoto_hip_w4_gemv would
 * write for x = that row. Block 0 also records the token as
 * aoto_hip_argmax_finish does (token_out, history, step state, RoPE rows) and
 * writes the raw embedding row to hidden_out (the step's residual stream; a
 * token outside the table stages and writes zeros and sets *error = 1). For the
 * block-staged q/k/v shapes (K = 896 or 4096, N <= 16384, norm weight
 * required) and at most aoto_hip_w4_gemv_finish_max_keys() keys; other shapes
 * return AOTO_ERR_UNSUPPORTED. */
size_t aoto_hip_w4_gemv_finish_max_keys(void);
int aoto_hip_w4_gemv_finish(const uint64_t* keys, int key_count, const void* embedding, int64_t embedding_rows,
                            const int32_t* words, const void* scales, const void* norm_weight, float eps,
                            const void* bias, float alpha, float beta, void* y, int K, int N, int group,
                            int64_t* token_out, int64_t* history, int* history_len, int32_t* step_state,
                            int capacity, const void* cos_table, const void* sin_table, int head_dim,
                            void* rope_rows, void* hidden_out, int* error, void* stream);

/* ---------------------------------------------------------------- generic graph kernels
 *
 * The compile_callable / compile_module plans (compiler.py:301-405 of the
 * reference: torch capture -> lowered graph -> one kernel per node) run on
 * these launchers. Tensors are described by aoto_tensor: a device pointer,
 * element type, shape and element strides (stride 0 broadcasts); data == NULL
 * with ndim 0 is a scalar operand holding `value`. Outputs are written through
 * their strides; shapes must match the op's rules (checked on the host). */

#define AOTO_MAX_DIMS 8

#define AOTO_DT_F32 0
#define AOTO_DT_BF16 1
#define AOTO_DT_I64 2
#define AOTO_DT_I32 3
#define AOTO_DT_BOOL 4
#define AOTO_DT_U8 5
#define AOTO_DT_I8 6

typedef struct aoto_tensor {
  void* data;
  int32_t dtype;
  int32_t ndim;
  int64_t shape[AOTO_MAX_DIMS];
  int64_t strides[AOTO_MAX_DIMS];
  double value;
} aoto_tensor;

/* Elementwise ops (runtime/mlx_ops/__init__.py:239-620 semantics): codes below
 * AOTO_EW_ADD take one operand, AOTO_EW_ADD..AOTO_EW_ISNAN two (ISNAN one),
 * AOTO_EW_WHERE three (cond, x, y). Float results compute in f32 and round
 * once to the output type; integer/bool outputs compute in int64; comparisons
 * compare exactly and write bool. */
#define AOTO_EW_CAST 0
#define AOTO_EW_NEG 1
#define AOTO_EW_ABS 2
#define AOTO_EW_RECIPROCAL 3
#define AOTO_EW_SQRT 4
#define AOTO_EW_RSQRT 5
#define AOTO_EW_EXP 6
#define AOTO_EW_LOG 7
#define AOTO_EW_SIGMOID 8
#define AOTO_EW_SILU 9
#define AOTO_EW_TANH 10
#define AOTO_EW_COS 11
#define AOTO_EW_SIN 12
#define AOTO_EW_RELU 13
#define AOTO_EW_GELU 14
#define AOTO_EW_GELU_TANH 15
#define AOTO_EW_ERF 16
#define AOTO_EW_FLOOR 17
#define AOTO_EW_CEIL 18
#define AOTO_EW_LOG1P 19
#define AOTO_EW_EXPM1 20
#define AOTO_EW_LOGICAL_NOT 21
#define AOTO_EW_BITWISE_NOT 22
#define AOTO_EW_ADD 32
#define AOTO_EW_SUB 33
#define AOTO_EW_MUL 34
#define AOTO_EW_DIV 35
#define AOTO_EW_DIV_TRUNC 36
#define AOTO_EW_DIV_FLOOR 37
#define AOTO_EW_POW 38
#define AOTO_EW_MAXIMUM 39
#define AOTO_EW_MINIMUM 40
#define AOTO_EW_REMAINDER 41
#define AOTO_EW_BIT_AND 42
#define AOTO_EW_BIT_OR 43
#define AOTO_EW_BIT_XOR 44
#define AOTO_EW_LOG_AND 45
#define AOTO_EW_LOG_OR 46
#define AOTO_EW_EQ 48
#define AOTO_EW_NE 49
#define AOTO_EW_LT 50
#define AOTO_EW_LE 51
#define AOTO_EW_GT 52
#define AOTO_EW_GE 53
#define AOTO_EW_ISNAN 54
#define AOTO_EW_WHERE 64

/* out (contiguous) = op(a, b, c) with numpy broadcasting of a, b, c to out's
 * shape; alpha scales b for ADD/SUB; unused operands may be NULL. */
int aoto_hip_generic_elementwise(int op, const aoto_tensor* out, const aoto_tensor* a, const aoto_tensor* b,
                                 const aoto_tensor* c, double alpha, void* stream);

/* Row reductions and scans over the last dim of `in` (its leading dims must
 * collapse to one stride): SUM, MEAN, AMAX, AMIN, ANY, ALL, ARGMAX, ARGMIN
 * write out[rows]; SOFTMAX, LOG_SOFTMAX, CUMSUM write out[rows, len].
 * (runtime/mlx_ops/__init__.py reductions; softmax in f32.) */
#define AOTO_RED_SUM 0
#define AOTO_RED_MEAN 1
#define AOTO_RED_AMAX 2
#define AOTO_RED_AMIN 3
#define AOTO_RED_ANY 4
#define AOTO_RED_ALL 5
#define AOTO_RED_ARGMAX 6
#define AOTO_RED_ARGMIN 7
#define AOTO_RED_SOFTMAX 8
#define AOTO_RED_LOG_SOFTMAX 9
#define AOTO_RED_CUMSUM 10
int aoto_hip_generic_reduce(int op, const aoto_tensor* out, const aoto_tensor* in, void* stream);

/* out[b] = alpha * a[b] . b[b] + beta * bias (bias broadcast by its strides,
 * or NULL); a [B, M, K], b [B, K, N], out [B, M, N], any strides, f32
 * accumulation (mm / bmm / addmm of the lowered graph). */
int aoto_hip_generic_matmul(const aoto_tensor* out, const aoto_tensor* a, const aoto_tensor* b,
                            const aoto_tensor* bias, float alpha, float beta, void* stream);

/* Advanced indexing of a contiguous source by index tensors over its leading
 * nidx dims (embedding, index.Tensor): the indices broadcast to out's leading
 * dims, the source's remaining dims follow. An index outside [-size, size)
 * sets *error (when non-NULL) to 1 and yields zeros. */
int aoto_hip_generic_index(const aoto_tensor* out, const aoto_tensor* src, int nidx,
                           const aoto_tensor* const* indices, int* error, void* stream);

/* dst = src (same shape, any strides, element-type conversion). */
int aoto_hip_generic_copy(const aoto_tensor* dst, const aoto_tensor* src, void* stream);

/* Contiguous dst[i] = start + i * step (step 0: a fill). */
int aoto_hip_generic_fill(const aoto_tensor* dst, double start, double step, void* stream);

/* The HF RMSNorm chain folded into one kernel (legalize/attention.py:332-525):
 * out = weight * cast_mid(float(x) * rsqrt(mean(float(x)^2) + eps)) over the
 * last dim of a contiguous x; weight may be NULL; mid_dtype is the element
 * type the normalized value is cast to before the weight multiply. */
int aoto_hip_generic_rms_norm(const aoto_tensor* out, const aoto_tensor* x, const aoto_tensor* weight, float eps,
                              int mid_dtype, void* stream);

/* scaled_dot_product_attention (legalize/attention.py:105-170): q [B, H, Lq, D],
 * k [B, Hk, Lk, D], v [B, Hk, Lk, Dv] (H % Hk == 0), mask broadcast to
 * [B, H, Lq, Lk] (bool keep / float additive) or NULL, is_causal; out
 * [B, H, Lq, Dv] contiguous; Lk <= 8192. Fully masked rows give zeros. */
int aoto_hip_generic_attention(const aoto_tensor* out, const aoto_tensor* q, const aoto_tensor* k,
                               const aoto_tensor* v, const aoto_tensor* mask, int causal, float scale,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AOTO_HIP_H */
