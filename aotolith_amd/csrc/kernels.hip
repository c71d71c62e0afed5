// The gfx950 code object of the W4 (and W8) decoder path: every kernel the C ABI
// (include/aoto_hip.h) launches, as extern "C" symbols looked up by name.
#include "common.h"
#include "w4_pack.h"
#include "w4_gemv.h"
#include "w4_gemv_stream.h"
#include "w4_gemv_rows.h"
#include "w4_gemm.h"
#include "w4_gemm_wide.h"
#include "w4_gemm_lds.h"
#include "w8.h"
#include "generic.h"
#include "decode.h"
#include "prefill.h"
#include "flash_attention.h"

// W4 decode GEMV: {lanes per row} x {norm prologue} x {paired} x {bias epilogue}.
AOTO_GEMV_LPR(0, 0, 0)
AOTO_GEMV_LPR(0, 0, 1)
AOTO_GEMV_LPR(1, 0, 0)
AOTO_GEMV_LPR(1, 0, 1)
AOTO_GEMV_LPR(0, 1, 0)
AOTO_GEMV_LPR(1, 1, 0)

// Wave-persistent streaming W4 GEMV: {lanes per row} x {chunks per lane} x
// {x vectors each lane stages, ceil(K / 512); 0 = each lane loads its own
// chunks directly} x {x held in registers}.
// K = 896: 8x4 for long outputs (single: x read from LDS; paired: x in
// registers), 32x1 direct for short paired ones (AOTO_GEMV_ROWS=0); K = 4096: 32x4.
AOTO_GEMV_STREAM_SINGLE(8, 4, 2, false)
AOTO_GEMV_STREAM_PAIRED(8, 4, 2, true)
AOTO_GEMV_STREAM_PAIRED(32, 1, 0, true)
AOTO_GEMV_STREAM_SINGLE(32, 4, 8, true)
AOTO_GEMV_STREAM_PAIRED(32, 4, 8, true)
// Multi-row direct GEMV for the paired gate/up at K = 896 (4 rows per lane; 2
// by AOTO_GEMV_ROWS): {lanes per row} x {chunks per lane} x {rows per lane}. (Measured and not
// kept: 8 rows per lane at K = 896, and 2 or 4 rows of a direct 64x3 layout
// at K = 4864, no faster than the streaming form.)
AOTO_GEMV_ROWS_SHAPE(32, 1, 2)
AOTO_GEMV_ROWS_SHAPE(32, 1, 4)
// Block-staged x for short or mid outputs: K = 896 (Qwen q/k/v, o) 32x1,
// K = 4096 (Llama-8B q/k/v, o, gate/up) 32x4, K = 4864 (Qwen down) 64x3,
// K = 14336 (Llama-8B down) 64x7. The single
// forms hold x in registers (same-process A/B, Llama-8B: down 10.9-11.3 -> 9.6-9.8
// us, q/k/v -0.1 us, o unchanged); the paired form reads it from LDS (no gain).
AOTO_GEMV_STREAM_BLOCKX_SINGLE(32, 1, 1)
AOTO_GEMV_STREAM_BLOCKX_SINGLE(32, 4, 2)
AOTO_GEMV_STREAM_BLOCKX_PAIRED(32, 4, 2)
AOTO_GEMV_STREAM_BLOCKX_SINGLE(64, 3, 3)
AOTO_GEMV_STREAM_BLOCKX_SINGLE(64, 7, 7)
// The greedy loop's first q/k/v GEMV of a step with the previous step's argmax
// finish in its prologue (K = 896: 32x1, K = 4096: 32x4; with and without bias).
AOTO_GEMV_STREAM_FINISH_KERNEL(32, 1, 1, 1, 1)
AOTO_GEMV_STREAM_FINISH_KERNEL(32, 1, 1, 1, 0)
AOTO_GEMV_STREAM_FINISH_KERNEL(32, 4, 2, 1, 1)
AOTO_GEMV_STREAM_FINISH_KERNEL(32, 4, 2, 1, 0)
// LM heads with the fused greedy-argmax keys: K = 896 (8x4), K = 4096 (32x4),
// and direct 64-lane forms for any other K up to 2048 / 6144.
AOTO_GEMV_STREAM_ARGMAX(8, 4, 2, false)
// the K = 896 and K = 4096 LM heads with their final norm, x staged once per block
// and copied into registers (same-process A/B, Qwen head 14.7-15.7 -> 14.0-14.1 us)
AOTO_GEMV_STREAM_KERNEL_X(aoto_w4_gemv_x8x4_n1_argmax, 8, 4, 1, true, 1, 0, 0, true, true)
AOTO_GEMV_STREAM_KERNEL_X(aoto_w4_gemv_x32x4_n1_argmax, 32, 4, 2, true, 1, 0, 0, true, true)
AOTO_GEMV_STREAM_ARGMAX(32, 4, 8, true)
AOTO_GEMV_STREAM_ARGMAX(64, 1, 0, true)
AOTO_GEMV_STREAM_ARGMAX(64, 3, 0, true)

// Prefill GEMM: {code width} x {n tiles per wave} x {m tiles per wave} x epilogue.
AOTO_GEMM_EPILOGUES(4, 1, 2)
AOTO_GEMM_EPILOGUES(4, 1, 4)
AOTO_GEMM_EPILOGUES(4, 1, 8)
AOTO_GEMM_EPILOGUES(4, 2, 4)
AOTO_GEMM_EPILOGUES(4, 2, 8)
AOTO_GEMM_EPILOGUES(8, 1, 2)
AOTO_GEMM_EPILOGUES(8, 1, 4)
AOTO_GEMM_EPILOGUES(8, 1, 8)
AOTO_GEMM_EPILOGUES(8, 2, 4)
AOTO_GEMM_EPILOGUES(8, 2, 8)
// The MLP's gate/up pair in one pass: {code width} x {n tiles} x {m tiles}.
AOTO_GEMM_PAIRED_INSTANCE(4, 1, 2)
AOTO_GEMM_PAIRED_INSTANCE(4, 1, 4)
AOTO_GEMM_PAIRED_INSTANCE(4, 1, 8)
AOTO_GEMM_PAIRED_INSTANCE(4, 2, 4)
AOTO_GEMM_PAIRED_INSTANCE(4, 2, 8)
AOTO_GEMM_PAIRED_INSTANCE(8, 1, 2)
AOTO_GEMM_PAIRED_INSTANCE(8, 1, 4)
AOTO_GEMM_PAIRED_INSTANCE(8, 1, 8)
AOTO_GEMM_PAIRED_INSTANCE(8, 2, 4)
AOTO_GEMM_PAIRED_INSTANCE(8, 2, 8)
// Long prefills, wide tiles (v_mfma_f32_32x32x16_bf16, LDS-staged): {code width} x
// {32-row tiles per wave} x {32-column tiles per wave} x {waves per block} x epilogue
// (the shapes whose staging buffers fit 160 KB of LDS).
AOTO_GEMM_WIDE_EPILOGUES(4, 4, 1, 4)
AOTO_GEMM_WIDE_EPILOGUES(4, 4, 2, 4)
AOTO_GEMM_WIDE_EPILOGUES(4, 4, 3, 4)
AOTO_GEMM_WIDE_EPILOGUES(4, 8, 1, 4)
AOTO_GEMM_WIDE_EPILOGUES(4, 4, 1, 8)
AOTO_GEMM_WIDE_EPILOGUES(8, 4, 1, 4)
AOTO_GEMM_WIDE_EPILOGUES(8, 4, 2, 4)
AOTO_GEMM_WIDE_EPILOGUES(8, 4, 1, 8)
AOTO_GEMM_WIDE_PAIRED_INSTANCE(4, 4, 1, 4)
AOTO_GEMM_WIDE_PAIRED_INSTANCE(8, 4, 1, 4)
// Long prefills whose grids fill whole rounds of 256 blocks: each packed tile
// expanded once per 256-row block into LDS (w4_gemm_lds.h), 8 waves of 64 x 64 or 64 x 96:
// {waves} x {32-row tiles per wave} x {32-column tiles per wave} x {bias} x {residual}.
AOTO_GEMM_LDS_INSTANCE(8, 2, 2, 0, 0)
AOTO_GEMM_LDS_INSTANCE(8, 2, 2, 1, 0)
AOTO_GEMM_LDS_INSTANCE(8, 2, 2, 0, 1)
AOTO_GEMM_LDS_INSTANCE(8, 2, 3, 0, 0)
AOTO_GEMM_LDS_INSTANCE(8, 2, 3, 1, 0)
AOTO_GEMM_LDS_INSTANCE(8, 2, 3, 0, 1)
AOTO_GEMM_LDS_PAIRED_INSTANCE(8, 2, 1)
AOTO_GEMM_LDS_PAIRED_INSTANCE(4, 2, 1)
AOTO_GEMM_LDS_PAIRED_COLUMN_INSTANCE(4, 1, 1)
AOTO_GEMM_LDS_SPLIT_INSTANCE(4, 1, 1, 1)
AOTO_GEMM_LDS_SPLIT_INSTANCE(4, 2, 2, 1)
// The q/k/v projection with bias, RoPE and cache fill: {code width} x {n tiles} x {m tiles} x {bias}.
AOTO_GEMM_ROPE_INSTANCE(4, 1, 2, 0)
AOTO_GEMM_ROPE_INSTANCE(4, 1, 2, 1)
AOTO_GEMM_ROPE_INSTANCE(4, 1, 4, 0)
AOTO_GEMM_ROPE_INSTANCE(4, 1, 4, 1)
AOTO_GEMM_ROPE_INSTANCE(4, 1, 8, 0)
AOTO_GEMM_ROPE_INSTANCE(4, 1, 8, 1)
AOTO_GEMM_ROPE_INSTANCE(4, 2, 4, 0)
AOTO_GEMM_ROPE_INSTANCE(4, 2, 4, 1)
AOTO_GEMM_ROPE_INSTANCE(4, 2, 8, 0)
AOTO_GEMM_ROPE_INSTANCE(4, 2, 8, 1)
AOTO_GEMM_ROPE_INSTANCE(8, 1, 2, 0)
AOTO_GEMM_ROPE_INSTANCE(8, 1, 2, 1)
AOTO_GEMM_ROPE_INSTANCE(8, 1, 4, 0)
AOTO_GEMM_ROPE_INSTANCE(8, 1, 4, 1)
AOTO_GEMM_ROPE_INSTANCE(8, 1, 8, 0)
AOTO_GEMM_ROPE_INSTANCE(8, 1, 8, 1)
AOTO_GEMM_ROPE_INSTANCE(8, 2, 4, 0)
AOTO_GEMM_ROPE_INSTANCE(8, 2, 4, 1)
AOTO_GEMM_ROPE_INSTANCE(8, 2, 8, 0)
AOTO_GEMM_ROPE_INSTANCE(8, 2, 8, 1)

// Eight-bit decode GEMV: {rows per wave} x {chunks per lane per pass}, with
// the decoder's epilogues (rms-norm prologue, paired gate/up, bias/residual).
AOTO_GEMV_W8_SHAPE(4, 1)
AOTO_GEMV_W8_SHAPE(2, 2)
AOTO_GEMV_W8_SHAPE(1, 4)

// Single-query attention (plain and RoPE-fused ring step): head dim.
// Decode attention: 4-wave blocks, {2, 4, 6, 8} K and V wave loads per wave
// (8-wave blocks measured no faster: 4.46 vs 4.38 us for the Qwen step).
AOTO_DECODE_ATTENTION_SHAPES(64, 4, 2, 4, 6, 8)
AOTO_DECODE_ATTENTION_SHAPES(128, 4, 2, 4, 6, 8)

// Prefill attention: head dim.
AOTO_FLASH_INSTANCE(64)
AOTO_FLASH_INSTANCE(128)
// short prompts at D = 64: 64 (32) queries per block, two 2-wave (1-wave) key groups
AOTO_FLASH_INSTANCE_KG(64, 2, false, _k2_q64, 1, 2)
AOTO_FLASH_INSTANCE_KG(64, 2, false, _k2_q32, 1, 1)
AOTO_FLASH_INSTANCE_KG(128, 2, false, _k2_q64, 1, 2)
