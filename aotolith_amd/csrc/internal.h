// Host-side helpers shared by the C-ABI sources of libaoto_hip.so (not part of the ABI).
#pragma once

namespace aoto {

// Record a printf-style message for aoto_hip_last_error() and return `code`.
int set_error(int code, const char* fmt, ...);

// Resolve, once per device and with that device current, the address of the
// allocation-free GEMM's static scratch buffer (noalloc.hip). Called when a code
// object is installed on the device.
void noalloc_prepare_device(int device);

// Automatic (0) tile / split codes of the unpaired 4-bit prefill GEMM (group size,
// gate epilogue or not) resolved to the explicit plan aoto_hip_w4_gemm runs
// (aoto_hip.cpp); other codes pass unchanged.
void resolve_gemm_codes(int M, int N, int K, int group, bool gate, int* tile, int* splits);

}  // namespace aoto
