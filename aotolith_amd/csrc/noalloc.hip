// The allocation-free prefill GEMM entry point (aoto_hip_w4_gemm_noalloc) and its
// static scratch buffer.
//
// aoto_hip_w4_gemm takes the split-K workspace from its caller; callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc) get this variant, whose split-K partials live in
// `scratch`: a file-scope device array the library holds on every GPU it runs on
// until the process ends. In host code `scratch` names a host-side stand-in, not
// device memory, so it is never passed to a kernel: each device's address is
// resolved once with hipGetSymbolAddress (with that device current, when its code
// object is installed) and only that address is used. The GEMM's split partials are
// stored (not accumulated), so nothing in the buffer needs clearing between calls.
// Calls on one GPU share its buffer: two calls that overlap in time on one device
// (different streams) race.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "aoto_hip.h"
#include "internal.h"

static __device__ __align__(256) unsigned char scratch[AOTO_HIP_NOALLOC_SCRATCH_BYTES];

namespace {

struct ScratchSlot {
  void* address = nullptr;
  hipError_t status = hipErrorNotInitialized;
};

std::mutex g_scratch_mutex;
std::map<int, ScratchSlot> g_scratch;  // device -> its copy of `scratch`

}  // namespace

namespace aoto {

void noalloc_prepare_device(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  ScratchSlot& slot = g_scratch[device];
  if (slot.address != nullptr) return;
  void* address = nullptr;
  slot.status = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
  slot.address = slot.status == hipSuccess ? address : nullptr;
}

}  // namespace aoto

extern "C" int aoto_hip_w4_gemm_noalloc(const void* x, const int32_t* words, const void* scales, const void* bias,
                                        const void* residual, const void* gate, void* y, int M, int N, int K,
                                        int group, int tile, int splits, void* stream) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return aoto::set_error(AOTO_ERR_HIP, "w4_gemm_noalloc: hipGetDevice: %s", hipGetErrorString(err));
  ScratchSlot slot;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    auto it = g_scratch.find(device);
    if (it != g_scratch.end()) slot = it->second;
  }
  if (slot.address == nullptr) {
    if (slot.status == hipErrorNotInitialized)
      return aoto::set_error(AOTO_ERR_NO_CODE_OBJECT, "w4_gemm_noalloc: no gfx950 code object loaded on device %d",
                             device);
    return aoto::set_error(AOTO_ERR_HIP, "w4_gemm_noalloc: scratch address on device %d: %s", device,
                           hipGetErrorString(slot.status));
  }
  // Automatic codes: the workspace entry point's plan, with its split count lowered
  // (to one at least) until the partials fit the scratch; explicit codes are kept
  // and refused if they do not fit.
  const bool automatic = tile == 0 && splits == 0;
  if (M > 0 && N > 0 && K > 0 && K % 64 == 0) aoto::resolve_gemm_codes(M, N, K, group, gate != nullptr, &tile, &splits);
  size_t need = aoto_hip_w4_gemm_workspace(M, N, K, tile, splits);
  if (automatic && need > AOTO_HIP_NOALLOC_SCRATCH_BYTES) {
    if (splits == 0) splits = (int)(need / ((size_t)M * N * sizeof(float)));  // the 16x16 plan's own count
    while (splits > 1 && need > AOTO_HIP_NOALLOC_SCRATCH_BYTES) need = aoto_hip_w4_gemm_workspace(M, N, K, tile, --splits);
  }
  if (need > AOTO_HIP_NOALLOC_SCRATCH_BYTES)
    return aoto::set_error(AOTO_ERR_UNSUPPORTED,
                           "w4_gemm_noalloc: this plan (M=%d N=%d K=%d tile=%d splits=%d) needs %zu bytes of split-K "
                           "partials and the static scratch holds %u; pass fewer splits, or call aoto_hip_w4_gemm "
                           "with a workspace", M, N, K, tile, splits, need, (unsigned)AOTO_HIP_NOALLOC_SCRATCH_BYTES);
  return aoto_hip_w4_gemm(x, words, scales, bias, residual, gate, y, M, N, K, group, tile, splits,
                          need > 0 ? slot.address : nullptr, stream);
}
