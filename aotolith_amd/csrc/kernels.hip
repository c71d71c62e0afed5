// The gfx950 code object of the W4 decoder path: every kernel the C ABI
// (include/aoto_hip.h) launches, as extern "C" symbols looked up by name.
#include "common.h"
#include "w4_pack.h"
#include "w4_gemv.h"
#include "w4_gemm.h"
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

// Prefill W4 GEMM: {n tiles per wave} x {m tiles per wave} x epilogue.
AOTO_GEMM_EPILOGUES(1, 4)
AOTO_GEMM_EPILOGUES(1, 8)
AOTO_GEMM_EPILOGUES(2, 4)
AOTO_GEMM_EPILOGUES(2, 8)

// Single-query attention: head dim x query heads per kv head.
AOTO_DECODE_ATTENTION_INSTANCE(64, 1)
AOTO_DECODE_ATTENTION_INSTANCE(64, 2)
AOTO_DECODE_ATTENTION_INSTANCE(64, 4)
AOTO_DECODE_ATTENTION_INSTANCE(64, 7)
AOTO_DECODE_ATTENTION_INSTANCE(64, 8)
AOTO_DECODE_ATTENTION_INSTANCE(128, 1)
AOTO_DECODE_ATTENTION_INSTANCE(128, 2)
AOTO_DECODE_ATTENTION_INSTANCE(128, 4)
AOTO_DECODE_ATTENTION_INSTANCE(128, 7)
AOTO_DECODE_ATTENTION_INSTANCE(128, 8)

// Prefill attention: head dim.
AOTO_FLASH_INSTANCE(64)
AOTO_FLASH_INSTANCE(128)
