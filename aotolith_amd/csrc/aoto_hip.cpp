// Host side of the C ABI declared in include/aoto_hip.h.
//
// Kernels live in a gfx950 code object (built from kernels.hip) that callers
// install per device with aoto_hip_load_code_object; every launcher checks its
// arguments against the kernel's limits on the host, looks its function up in
// the current device's module and enqueues it with hipModuleLaunchKernel on the
// caller's stream. No allocation, no synchronization, no per-call state.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>

#include "aoto_hip.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buf, sizeof(buf), fmt, args);
  va_end(args);
  g_error = buf;
  return code;
}

struct DeviceModule {
  hipModule_t module = nullptr;
  std::unordered_map<std::string, hipFunction_t> functions;
};

std::mutex g_mutex;
std::map<int, DeviceModule> g_modules;

int current_device(int* device) {
  hipError_t err = hipGetDevice(device);
  if (err != hipSuccess) return fail(AOTO_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(err));
  return AOTO_OK;
}

int lookup(const char* name, hipFunction_t* fn) {
  int device = 0;
  if (int s = current_device(&device)) return s;
  std::lock_guard<std::mutex> lock(g_mutex);
  auto it = g_modules.find(device);
  if (it == g_modules.end() || it->second.module == nullptr)
    return fail(AOTO_ERR_NO_CODE_OBJECT, "no gfx950 code object loaded on device %d", device);
  auto& fns = it->second.functions;
  auto found = fns.find(name);
  if (found != fns.end()) {
    *fn = found->second;
    return AOTO_OK;
  }
  hipFunction_t f = nullptr;
  hipError_t err = hipModuleGetFunction(&f, it->second.module, name);
  if (err != hipSuccess)
    return fail(AOTO_ERR_NO_CODE_OBJECT, "kernel %s not found in the code object: %s", name,
                hipGetErrorString(err));
  fns.emplace(name, f);
  *fn = f;
  return AOTO_OK;
}

template <typename... Args>
int launch(const char* name, dim3 grid, dim3 block, unsigned shared, void* stream, Args... args) {
  hipFunction_t fn = nullptr;
  if (int s = lookup(name, &fn)) return s;
  void* params[] = {static_cast<void*>(&args)...};
  hipError_t err = hipModuleLaunchKernel(fn, grid.x, grid.y, grid.z, block.x, block.y, block.z, shared,
                                         static_cast<hipStream_t>(stream), params, nullptr);
  if (err != hipSuccess) return fail(AOTO_ERR_HIP, "launch %s: %s", name, hipGetErrorString(err));
  return AOTO_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" {

int aoto_hip_abi_version(void) { return AOTO_HIP_ABI_VERSION; }

size_t aoto_hip_last_error(char* buf, size_t size) {
  if (buf != nullptr && size > 0) {
    size_t n = g_error.size() < size - 1 ? g_error.size() : size - 1;
    memcpy(buf, g_error.data(), n);
    buf[n] = '\0';
  }
  return g_error.size();
}

int aoto_hip_load_code_object(const void* image, size_t size) {
  if (image == nullptr || size == 0) return fail(AOTO_ERR_ARGUMENT, "empty code object");
  int device = 0;
  if (int s = current_device(&device)) return s;
  hipModule_t module = nullptr;
  hipError_t err = hipModuleLoadData(&module, image);
  if (err != hipSuccess)
    return fail(AOTO_ERR_HIP, "hipModuleLoadData (%zu bytes): %s", size, hipGetErrorString(err));
  std::lock_guard<std::mutex> lock(g_mutex);
  auto& slot = g_modules[device];
  if (slot.module != nullptr) hipModuleUnload(slot.module);
  slot.module = module;
  slot.functions.clear();
  return AOTO_OK;
}

int aoto_hip_unload_code_object(void) {
  int device = 0;
  if (int s = current_device(&device)) return s;
  std::lock_guard<std::mutex> lock(g_mutex);
  auto it = g_modules.find(device);
  if (it != g_modules.end()) {
    if (it->second.module != nullptr) hipModuleUnload(it->second.module);
    g_modules.erase(it);
  }
  return AOTO_OK;
}

int aoto_hip_code_object_loaded(void) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(g_mutex);
  auto it = g_modules.find(device);
  return (it != g_modules.end() && it->second.module != nullptr) ? 1 : 0;
}

int aoto_hip_w4_quantize(const void* weight, int weight_is_f32, int rows, int inner, int group,
                         int32_t* packed, void* scales_bf16, float* scales_f32, void* stream) {
  if (!weight || !packed || !scales_bf16) return fail(AOTO_ERR_ARGUMENT, "w4_quantize: null pointer");
  if (rows <= 0 || inner <= 0) return fail(AOTO_ERR_ARGUMENT, "w4_quantize: empty shape %dx%d", rows, inner);
  if (group <= 0 || group % 8 != 0 || inner % group != 0)
    return fail(AOTO_ERR_ARGUMENT, "w4_quantize: group %d must be a positive multiple of 8 dividing %d",
                group, inner);
  long long tasks = (long long)rows * (inner / group);
  unsigned blocks = (unsigned)((tasks + 255) / 256);
  return launch("aoto_w4_quantize", dim3(blocks), dim3(256), 0, stream, weight, weight_is_f32, rows, inner,
                group, packed, scales_bf16, scales_f32);
}

int aoto_hip_w4_dequantize(const int32_t* packed, const void* scales, int rows, int inner, int group,
                           void* out, void* stream) {
  if (!packed || !scales || !out) return fail(AOTO_ERR_ARGUMENT, "w4_dequantize: null pointer");
  if (rows <= 0 || inner <= 0 || inner % 8 != 0)
    return fail(AOTO_ERR_ARGUMENT, "w4_dequantize: bad shape %dx%d", rows, inner);
  if (group <= 0 || group % 8 != 0 || inner % group != 0)
    return fail(AOTO_ERR_ARGUMENT, "w4_dequantize: bad group %d for inner %d", group, inner);
  if (!aligned16(out)) return fail(AOTO_ERR_ARGUMENT, "w4_dequantize: output must be 16-byte aligned");
  long long words = (long long)rows * (inner / 8);
  unsigned blocks = (unsigned)((words + 255) / 256);
  return launch("aoto_w4_dequantize", dim3(blocks), dim3(256), 0, stream, packed, scales, rows, inner, group,
                out);
}

int aoto_hip_w4_gemv(const void* x, const int32_t* words, const void* scales, const int32_t* up_words,
                     const void* up_scales, const void* norm_weight, float eps, const void* bias, float alpha,
                     float beta, void* y, int K, int N, int group, int lanes_per_row, void* stream) {
  if (!x || !words || !scales || !y) return fail(AOTO_ERR_ARGUMENT, "w4_gemv: null pointer");
  if ((up_words == nullptr) != (up_scales == nullptr))
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv: paired projection needs both up_words and up_scales");
  const bool paired = up_words != nullptr;
  if (paired && bias != nullptr)
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv: the paired epilogue takes no bias");
  if (N <= 0 || K <= 0) return fail(AOTO_ERR_ARGUMENT, "w4_gemv: empty shape K=%d N=%d", K, N);
  if (K % 32 != 0 || group <= 0 || group % 32 != 0 || K % group != 0 || K > 32768)
    return fail(AOTO_ERR_UNSUPPORTED, "w4_gemv: needs K %% 32 == 0, group %% 32 == 0 dividing K, K <= 32768 "
                "(K=%d group=%d)", K, group);
  if (!aligned16(x) || !aligned16(words) || (up_words && !aligned16(up_words)) ||
      (norm_weight && !aligned16(norm_weight)))
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv: x, words and norm weight must be 16-byte aligned");
  int lpr = lanes_per_row;
  if (lpr == 0) {
    // Fill the chip first (>= 2 blocks per CU on 256 CUs), then keep at least two
    // 16-byte chunks per lane so each lane has loads in flight.
    const int chunks = K / 32;
    lpr = 4;
    while (lpr < 64) {
      const long long blocks = ((long long)N + (4 * 64 / lpr) - 1) / (4 * 64 / lpr);
      if (blocks >= 512 || chunks / (lpr * 2) < 2) break;
      lpr *= 2;
    }
  }
  if (lpr != 4 && lpr != 8 && lpr != 16 && lpr != 32 && lpr != 64)
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv: lanes_per_row must be 4, 8, 16, 32 or 64 (got %d)", lpr);
  const int rows_per_block = 4 * (64 / lpr);
  const unsigned blocks = (unsigned)((N + rows_per_block - 1) / rows_per_block);
  const unsigned shared = (unsigned)((K / 8) * 16 + (K / 32) * 4);
  const int norm = norm_weight != nullptr;
  const int has_bias = bias != nullptr;
  char name[64];
  snprintf(name, sizeof(name), "aoto_w4_gemv_l%d_n%d_p%d_b%d", lpr, norm, paired ? 1 : 0, has_bias);
  return launch(name, dim3(blocks), dim3(256), shared, stream, x, words, scales, up_words, up_scales,
                norm_weight, eps, bias, alpha, beta, y, K, N, group);
}

}  // extern "C"
