// Host-side helpers shared by the C-ABI sources of libaoto_hip.so (not part of the ABI).
#pragma once

namespace aoto {

// Record a printf-style message for aoto_hip_last_error() and return `code`.
int set_error(int code, const char* fmt, ...);

// Resolve, once per device and with that device current, the address of the
// allocation-free GEMM's static scratch buffer (noalloc.hip). Called when a code
// object is installed on the device.
void noalloc_prepare_device(int device);

// Where automatic (0) tile / split codes of the unpaired prefill GEMM would take
// the long-prefill library path, resolve them to the fused kernel's own plan
// (aoto_hip.cpp), for callers without room for the unpacked weight.
void fused_gemm_codes(int M, int N, int K, int* tile, int* splits);

// Plain bf16 GEMMs on hipBLASLt (blaslt.cpp): D[M][N] = X[M][K] . W[N][K]^T
// (+ bias[N]) (+ c[M][N]), f32 accumulation, D bf16 or f32. library_prepare
// creates the device's handle (called when a code object is installed, outside
// any graph capture); library_gemm enqueues one GEMM on `stream`. `scratch`
// (M * N of the output type, not aliasing the operands) takes the candidate
// timing of a shape's first uncaptured call; its contents are overwritten.
int library_prepare(int device);
int library_gemm(int M, int N, int K, const void* x, const void* w, const void* bias, const void* c, void* d,
                 bool d_f32, void* scratch, void* stream);

}  // namespace aoto
