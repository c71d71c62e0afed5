// The gfx950 code object of the W4 decoder path: every kernel the C ABI
// (include/aoto_hip.h) launches, as extern "C" symbols looked up by name.
#include "common.h"
#include "w4_pack.h"
#include "w4_gemv.h"

// W4 decode GEMV: {lanes per row} x {norm prologue} x {paired} x {bias epilogue}.
AOTO_GEMV_LPR(0, 0, 0)
AOTO_GEMV_LPR(0, 0, 1)
AOTO_GEMV_LPR(1, 0, 0)
AOTO_GEMV_LPR(1, 0, 1)
AOTO_GEMV_LPR(0, 1, 0)
AOTO_GEMV_LPR(1, 1, 0)
