// Host side of the C ABI declared in include/aoto_hip.h.
//
// Kernels live in a gfx950 code object (built from kernels.hip) that callers
// install per device with aoto_hip_load_code_object; every launcher checks its
// arguments against the kernel's limits on the host, looks its function up in
// the current device's module and enqueues it with hipModuleLaunchKernel on the
// caller's stream. No allocation, no synchronization, no per-call state.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "aoto_hip.h"
#include "gemm_args.h"
#include "generic_args.h"
#include "internal.h"
#include "gemv_finish_args.h"


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

}  // namespace

int aoto::set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buf, sizeof(buf), fmt, args);
  va_end(args);
  g_error = buf;
  return code;
}

namespace {

struct DeviceModule {
  hipModule_t module = nullptr;
  std::unordered_map<std::string, hipFunction_t> functions;
  // Modules replaced by a later load while captured graphs were held: such a
  // graph holds their kernel handles, and replaying it after an unload would
  // execute freed code (a GPU memory fault). Released when the last hold goes.
  std::vector<hipModule_t> retired;
};

std::mutex g_mutex;
std::map<int, DeviceModule> g_modules;
// Captured HIP graphs (process-wide) whose nodes launch kernels of the loaded
// modules: aoto_hip_hold_graphs(+1 / -1). While any is held, no module is unloaded.
int g_graph_holds = 0;

// With g_mutex held and no graph held: unload every retired module (after the
// device's queued work, which may still run their kernels).
void release_retired_locked() {
  for (auto& entry : g_modules) {
    if (entry.second.retired.empty()) continue;
    int current = 0;
    hipGetDevice(&current);
    hipSetDevice(entry.first);
    hipDeviceSynchronize();
    for (hipModule_t old : entry.second.retired) hipModuleUnload(old);
    entry.second.retired.clear();
    hipSetDevice(current);
  }
}

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

// Kernel symbols launched by this thread while recording is on (aoto_hip_trace_launches),
// newline-separated, for plans that name the kernels they run.
thread_local bool g_trace = false;
thread_local std::string g_trace_names;

void trace_launch(const char* name) {
  if (g_trace) {
    g_trace_names += name;
    g_trace_names += '\n';
  }
}

template <typename... Args>
int launch(const char* name, dim3 grid, dim3 block, unsigned shared, void* stream, Args... args) {
  hipFunction_t fn = nullptr;
  if (int s = lookup(name, &fn)) return s;
  void* params[] = {static_cast<void*>(&args)...};
  hipError_t err = hipModuleLaunchKernel(fn, grid.x, grid.y, grid.z, block.x, block.y, block.z, shared,
                                         static_cast<hipStream_t>(stream), params, nullptr);
  if (err != hipSuccess) return fail(AOTO_ERR_HIP, "launch %s: %s", name, hipGetErrorString(err));
  trace_launch(name);
  return AOTO_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// Compute units of the current device (cached per device).
int cu_count() {
  static std::mutex mutex;
  static std::map<int, int> counts;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mutex);
  auto it = counts.find(device);
  if (it != counts.end()) return it->second;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0) n = 256;
  counts[device] = n;
  return n;
}

// Persistent GEMV blocks per CU: the shape's own default unless
// AOTO_GEMV_BLOCKS_PER_CU overrides it (read once).
int gemv_blocks_per_cu(int shape_default) {
  static int value = [] {
    const char* env = getenv("AOTO_GEMV_BLOCKS_PER_CU");
    return env ? atoi(env) : 0;
  }();
  return value > 0 ? value : shape_default;
}

// Streaming GEMV instance for a reduction length and output count: lanes per
// row, chunks per lane, and whether each lane loads its own x chunks (direct,
// no LDS) or the wave stages x into LDS first. Short outputs (a decoder
// layer's projections) are latency-bound and get 32-64 lanes per row with
// direct x loads; long outputs (LM heads) get few lanes per row and one staged
// copy of x per wave. The paired gate/up form needs two weight sets in
// registers, so it uses a narrower per-lane share at K = 896.
// Must agree with the instances in kernels.hip.
struct StreamShape {
  int lpr, cpl;
  bool direct;
  int blocks_per_cu = 2;  // persistent 4-wave blocks per CU
  bool block_x = false;   // x staged once per 4-wave block (aoto_w4_gemv_x* instances)
  int rows = 0;           // > 0: the multi-row direct form, rows per lane (aoto_w4_gemv_r* instances)
};

// Rows per lane of the multi-row direct GEMV; AOTO_GEMV_ROWS overrides the
// shape's default (0 selects the streaming form) where that instance exists.
int gemv_rows(int lpr, int shape_default) {
  static const int value = [] {
    const char* env = getenv("AOTO_GEMV_ROWS");
    return env ? atoi(env) : -1;
  }();
  if (value < 0) return shape_default;
  if (value == 0) return 0;
  const bool exists = lpr == 32 && (value == 2 || value == 4);
  return exists ? value : shape_default;
}

bool stream_shape(int K, int N, bool paired, StreamShape* s) {
  const bool short_out = N <= 8192;
  switch (K) {
    case 896:
      // Long outputs: 8 lanes x 4 chunks (32 slots for the 28 chunks of a row;
      // the 4 spare slots repeat the last chunk), x read from LDS so the two
      // weight register sets fit; 2 blocks per CU - each wave then takes ~9 row
      // tiles, over which its x staging and pipeline fill and drain amortize
      // (greedy loop's LM-head kernel, 151936 rows, 1 / 2 / 3 / 4 / 5 / 6 / 8
      // blocks per CU: 16.7 / 14.9 / 15.5 / 16.0 / 16.8 / 17.0 / 17.5 us).
      // Short outputs, paired gate/up: the multi-row direct form, one normalized
      // copy of x per lane serving 4 rows (3.9 vs 4.3 us for Qwen's 2 x 4864 rows).
      // Single projections (q/k/v, o): one copy of x per 4-wave block, held in
      // registers - in the direct forms every wave loaded all of x and the norm
      // weight, more bytes per CU than its weights (Qwen q/k/v 2.87 -> 2.74 us, o
      // 2.91 -> 2.51, decode 2385-2391 -> 2414-2417 tok/s in alternating runs on
      // one box; the paired form this way: 4.15 -> 4.40 us).
      if (short_out && paired) {
        *s = {32, 1, true};
        s->rows = gemv_rows(32, 4);
      } else if (short_out) {
        *s = {32, 1, false, 1, true};
      } else
        *s = paired ? StreamShape{8, 4, false} : StreamShape{8, 4, false, 2};
      return true;
    case 4096:
      // Up to 16384 outputs (q/k/v, o, gate/up of an 8B model) a wave holds too
      // few row tiles to amortize its own copy of x: one copy per block, and one
      // block per CU - every block stages all of x, so fewer blocks move fewer
      // bytes (Llama-8B, 1 / 2 / 3 / 4 blocks per CU: gate/up 14.8 / 16.3 / 17.1 /
      // 16.8 us, q/k/v 5.39 / 5.46 / 5.84 / 5.80, o 4.14-4.18).
      if (N <= 16384)
        *s = {32, 4, false, 1, true};
      else
        *s = {32, 4, false};
      return true;
    case 4864:
      // One copy of x per 4-wave block, held in registers: the direct form had
      // every wave load all 9.7 KB of x, ~40 KB per CU beside ~9 KB of weights
      // (Qwen down projection 3.58 -> 3.29 us, decode 2345-2359 -> 2379-2382
      // tok/s in alternating runs on one box).
      if (paired || !short_out) return false;
      *s = {64, 3, false, 1, true};
      return true;
    case 14336:
      // 28 KB of x per block: one block per CU (down projection 10.28 against
      // 10.75 us at two).
      if (paired) return false;
      *s = {64, 7, false, 1, true};
      return true;
    default:
      // Other reductions use the block-staged kernel.
      return false;
  }
}

// Launch geometry of a streaming GEMV: one wave per tile of 64/lpr rows up to
// the wave budget (CUs x blocks-per-CU x 4); grids no larger than the CU count
// use 1-wave blocks so every wave gets its own CU.
struct StreamLaunch {
  long long grid;
  int wpb;
  unsigned shared;  // LDS bytes per block
  int shift;        // log2(group / 32)
};

StreamLaunch stream_launch(const StreamShape& ss, int K, int N, int group) {
  const long long tiles = ((long long)N + (64 / ss.lpr) - 1) / (64 / ss.lpr);
  const long long budget = (long long)cu_count() * gemv_blocks_per_cu(ss.blocks_per_cu) * 4;
  const long long waves = tiles < budget ? tiles : budget;
  StreamLaunch l{};
  // block-staged x needs full 4-wave blocks (the staging splits x over 256 threads)
  l.wpb = (waves <= cu_count() && !ss.block_x) ? 1 : 4;
  l.grid = (waves + l.wpb - 1) / l.wpb;
  // Direct instances read no LDS; staged ones need one region per wave, or one
  // per block when x is shared.
  const unsigned region = ss.direct ? 0u : (unsigned)((K / 8) * 16 + ((K / 32 + 3) / 4) * 16);
  l.shared = ss.block_x ? region : region * l.wpb;
  while ((32 << l.shift) < group) ++l.shift;
  return l;
}

// Lane layout of the LM-head GEMV with fused argmax keys: the streaming shape
// when there is one, else a direct 64-lane form for K up to 6144.
bool argmax_shape(int K, int N, int group, StreamShape* s) {
  if (K % 32 != 0 || group <= 0 || group % 32 != 0 || (group & (group - 1)) != 0 || K % group != 0 ||
      (K / group) % 2 != 0)
    return false;
  // (the 32x1 direct and the block-staged shapes have no argmax instance)
  if (stream_shape(K, N, false, s) && !(s->direct && s->lpr == 32) && !s->block_x) {
    s->rows = 0;  // the argmax instances are streaming ones
    return true;
  }
  if (K <= 64 * 32) {
    *s = {64, 1, true};
    return true;
  }
  if (K <= 64 * 3 * 32) {
    *s = {64, 3, true};
    return true;
  }
  return false;
}

unsigned blocks_for(long long items, int threads) { return (unsigned)((items + threads - 1) / threads); }

// Decode attention split choice. One block holds at most `max_chunk` keys (8
// wave loads of 64/(D/8) rows per wave, 4 waves); longer windows split into blocks whose
// records a merge launch combines. `requested` > 0 asks for that many splits.
int decode_max_chunk(int head_dim) { return head_dim == 64 ? 256 : 128; }

// Block size and loads per wave of a decode-attention launch: 4 waves, each
// issuing J wave loads (512/D key rows each) of K and of V; J is the smallest
// instance (2, 4, 6 or 8) that covers the chunk, so no load is idle when the
// chunk is a multiple of 4 * 2 * 512/D keys (Qwen's 192-key window: J = 6,
// 4.38 us against 4.63 for J = 8 on MI355X).
struct AttnShape {
  int waves, loads;
};
AttnShape attention_shape(int head_dim, int chunk) {
  const int waves = 4;
  const int per_load = waves * (512 / head_dim);
  int j = (chunk + per_load - 1) / per_load;
  j = j < 2 ? 2 : j + (j & 1);
  return {waves, j};
}

void decode_split(int head_dim, int capacity, int requested, long long rows, int* splits, int* chunk) {
  const int most = decode_max_chunk(head_dim);
  int s = requested > 0 ? requested : (capacity + most - 1) / most;
  if (requested <= 0 && s > 1) {
    // A window that needs a merge launch anyway is spread over ~768 blocks,
    // chunks of at least 32 keys (Llama-8B, 32 heads, split + merge per layer:
    // 768-key window 8.5 us at 12 or 24 splits, 9.3 at 6; 2304-key window 10.8 us
    // at 24 splits, 11.8 at 36, 13.4 at 48, 13.6 at 18).
    const long long want = (768 + rows - 1) / rows;
    const int finest = (capacity + 31) / 32;
    if (want > s) s = (int)(want < finest ? want : finest);
  }
  int c = (capacity + s - 1) / s;
  if (c > most) c = most;
  s = (capacity + c - 1) / c;
  *splits = s;
  *chunk = c;
}

}  // namespace

extern "C" {

int aoto_hip_abi_version(void) { return AOTO_HIP_ABI_VERSION; }

int aoto_hip_trace_launches(int enable) {
  const int previous = g_trace ? 1 : 0;
  g_trace = enable != 0;
  if (g_trace && !previous) g_trace_names.clear();
  return previous;
}

size_t aoto_hip_take_launches(char* buf, size_t size) {
  const size_t n = g_trace_names.size();
  if (buf != nullptr && size > 0) {
    const size_t copied = n < size - 1 ? n : size - 1;
    memcpy(buf, g_trace_names.data(), copied);
    buf[copied] = '\0';
    if (copied == n) g_trace_names.clear();
  }
  return n;
}

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
  if (slot.module != nullptr) slot.retired.push_back(slot.module);
  slot.module = module;
  slot.functions.clear();
  aoto::noalloc_prepare_device(device);
  if (g_graph_holds == 0) release_retired_locked();
  return AOTO_OK;
}

int aoto_hip_hold_graphs(int delta) {
  std::lock_guard<std::mutex> lock(g_mutex);
  if (delta == 0 || g_graph_holds + delta < 0)
    return fail(AOTO_ERR_ARGUMENT, "hold_graphs: %d held, cannot change by %d", g_graph_holds, delta);
  g_graph_holds += delta;
  if (g_graph_holds == 0) release_retired_locked();
  return AOTO_OK;
}

int aoto_hip_graph_holds(void) {
  std::lock_guard<std::mutex> lock(g_mutex);
  return g_graph_holds;
}

int aoto_hip_unload_code_object(void) {
  {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_graph_holds > 0)
      return fail(AOTO_ERR_ARGUMENT, "unload_code_object: %d captured graphs still launch kernels of the loaded "
                  "code objects; release them (aoto_hip_hold_graphs(-1)) first", g_graph_holds);
  }
  int device = 0;
  if (int s = current_device(&device)) return s;
  std::lock_guard<std::mutex> lock(g_mutex);
  auto it = g_modules.find(device);
  if (it != g_modules.end()) {
    if (it->second.module != nullptr) hipModuleUnload(it->second.module);
    for (hipModule_t old : it->second.retired) hipModuleUnload(old);
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
  const int norm = norm_weight != nullptr;
  const int has_bias = bias != nullptr;
  const unsigned shared = (unsigned)((K / 8) * 16 + (K / 32) * 4);
  StreamShape ss{};
  const bool pow2_group = (group & (group - 1)) == 0;
  // The streaming form reads scales and bias as aligned 32-bit pairs.
  const bool pairs_ok = (K / group) % 2 == 0 && aligned4(scales) && (!up_scales || aligned4(up_scales)) &&
                        (!bias || (N % 2 == 0 && aligned4(bias)));
  // (the multi-row instances take 64-code groups; other groups use the streaming form)
  if (lanes_per_row == 0 && pairs_ok && group == 64 && stream_shape(K, N, paired, &ss) && ss.rows > 0) {
    // one 1-wave block per tile of (64 / lpr) * rows rows
    const int rows_per_wave = (64 / ss.lpr) * ss.rows;
    const unsigned grid = (unsigned)((N + rows_per_wave - 1) / rows_per_wave);
    char rname[64];
    snprintf(rname, sizeof(rname), "aoto_w4_gemv_r%dx%dx%d_n%d_p%d_b%d", ss.lpr, ss.cpl, ss.rows, norm,
             paired ? 1 : 0, has_bias);
    return launch(rname, dim3(grid), dim3(64), 0u, stream, words, scales, up_words, up_scales, x, norm_weight, K,
                  N, bias, eps, alpha, beta, y);
  }
  if (lanes_per_row == 0 && pow2_group && pairs_ok && stream_shape(K, N, paired, &ss)) {
    const StreamLaunch l = stream_launch(ss, K, N, group);
    char sname[64];
    snprintf(sname, sizeof(sname), "aoto_w4_gemv_%c%dx%d_n%d_p%d_b%d", ss.block_x ? 'x' : 's', ss.lpr, ss.cpl,
             norm, paired ? 1 : 0, has_bias);
    unsigned long long* no_keys = nullptr;
    return launch(sname, dim3((unsigned)l.grid), dim3(64 * l.wpb), l.shared, stream, words, scales, x, norm_weight,
                  K, N, l.shift, l.wpb, bias, up_words, up_scales, eps, alpha, beta, y, no_keys);
  }
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
  char name[64];
  snprintf(name, sizeof(name), "aoto_w4_gemv_l%d_n%d_p%d_b%d", lpr, norm, paired ? 1 : 0, has_bias);
  return launch(name, dim3(blocks), dim3(256), shared, stream, x, words, scales, up_words, up_scales,
                norm_weight, eps, bias, alpha, beta, y, K, N, group);
}

namespace {

// Prefill GEMM launch plan: tile shape and split-K count. Small grids (the
// M = 128 prefill of a 0.5B model gives 14-76 output tiles) split the
// reduction so at least ~256 blocks run; each slice keeps >= 2 k-steps of 64.
struct GemmPlan {
  int tn, tm, splits, kslice;
  // the wide-tile family (w4_gemm_wide.h): 32-row / 32-column tiles per wave, waves per block
  int wide_mt = 0, wide_nt = 0, wide_nw = 0;
  // the dequant-once family (w4_gemm_lds.h): lds_waves waves, lds_bm-row blocks of
  // lds_bn columns per weight
  bool lds = false;
  int lds_bm = 0, lds_bn = 0, lds_waves = 0;
  int bm() const { return lds ? lds_bm : wide_mt ? 32 * wide_mt : 16 * tm; }
  int bn() const { return lds ? lds_bn : wide_nt ? wide_nw * 32 * wide_nt : 64 * tn; }
  int threads() const { return lds ? 64 * lds_waves : wide_nw ? 64 * wide_nw : 256; }
};

// Wide-tile codes: 100 * (waves per block / 2) + 10 * (32-row tiles per wave) +
// (32-column tiles per wave), the waves side by side along n (w4_gemm_wide.h).
bool wide_code(int tile) {
  return tile == 241 || tile == 242 || tile == 243 || tile == 281 || tile == 441;
}

// Dequant-once codes (w4_gemm_lds.h, 4-bit codes, unsplit): 822 / 823 = 8 waves of
// 64 x 64 / 64 x 96 (256 x 128 / 256 x 192 blocks), 821 = the paired gate/up form
// (256 x (64 + 64) blocks); for short prompts the paired form on 128-row blocks of
// 4 waves, 812 = 64 x (32 + 32) per wave (128 x (64 + 64) blocks), 811 = 32 x (32 + 32)
// per wave, one wave along n (128 x (32 + 32) blocks).
// 813 / 814 = the single form's split-K partials on 128-row blocks of 4 waves, 128 x 32
// (one wave along n, 32 x 32 per wave) / 128 x 64 (64 x 32 per wave) blocks, summed and
// given their epilogue by the split reduce kernels (at any split count, 1 included).
bool lds_code(int tile) {
  return tile == 811 || tile == 812 || tile == 813 || tile == 814 || tile == 821 || tile == 822 || tile == 823;
}
bool lds_paired_code(int tile) { return tile == 811 || tile == 812 || tile == 821; }
bool lds_split_code(int tile) { return tile == 813 || tile == 814; }

// The automatic plan's choice of the dequant-once kernel (its tile code, or 0):
// 4-bit codes, a power-of-two group with an even count per row, no gate epilogue,
// and a grid whose last round of 256 blocks (one per CU) is at least 90% full - 128
// columns per block where that fills the rounds, else 192. Each packed tile is
// expanded once per 256-row block instead of once per 128-row wave, which pays where
// the rounds are full: measured on MI355X at 2048 rows (Llama-3-8B, same process,
// us): gate/up 484 against 513-528 for the paired 241, o 75 against 81 and down 232
// against 241 for 441.
//
// Short prompts (32-256 rows), the paired gate/up only: 128-row blocks of 4 waves,
// 64 + 64 columns (812) where that gives at least 128 blocks (from 65 rows), else
// 32 + 32 (811) where that fits one round of 256 blocks. Every wave of the 16x16
// kernel those replace expands its own columns' words; here the four row waves share
// one expansion. Measured on MI355X (us, automatic plan -> dequant-once): K = 896 ->
// 2 x 4864 at 32 / 64 / 128 / 256 rows 11.0 / 14.4 / 11.4 / 17.4 -> 9.6 / 9.6 / 9.6
// (811) / 14.0 (812); K = 4096 -> 2 x 14336 at 128 / 256 rows 61.8 / 90.2 -> 47.8 /
// 88.6 (812), at 64 rows 40.1 against 47.7 (kept on the 16x16 kernel).
//
// Short prompts, single projections with long reductions (K >= 2048: down, and o at
// 8B widths) and no RoPE epilogue: the split-K form, 128 x 64 blocks (814) where
// those give >= 64 column blocks, else 128 x 32 (813), split to ~232 blocks and summed
// with the epilogue by the 16x16 kernel's reduce launches. Measured on MI355X (us,
// with the residual + next-RMSNorm reduce): 4864 -> 896 at 64 / 128 / 256 rows 9.8 /
// 12.1 / 23.2 -> 9.7 / 10.7 / 13.5 (813); 4096 -> 4096 at 64 / 128 / 256 rows 24.4 /
// 25.7 / 29.1 -> 15.1 / 17.9 / 22.3 (814); 14336 -> 4096 at 128 rows 65.9 -> 31.4; at
// K = 896 (0.5B o, q/k/v) the 16x16 plan stays (7.3 / 7.8 against 7.5 / 7.8 at best).
int lds_short_single(int M, int N, int K) {
  if (M < 32 || M > 256 || K < 2048 || K % 64 != 0) return 0;
  return (long long)((N + 63) / 64) * ((M + 127) / 128) >= 64 ? 814 : 813;
}

int lds_auto(int bits, int M, int N, int K, int group, bool paired, bool gate, bool rope) {
  if (bits != 4 || gate || K % 64 != 0 || (group & (group - 1)) != 0 || group < 32 || (K / group) % 2 != 0)
    return 0;
  // the kernel's per-lane load offsets are 32-bit
  if ((long long)M * K * 2 >= (1LL << 31) || (long long)N * K / 2 >= (1LL << 31)) return 0;
  if (M < 1024) {
    if (!paired) return rope ? 0 : lds_short_single(M, N, K);
    if (M < 32 || M > 256) return 0;
    const long long mb = (M + 127) / 128;
    if (M > 64 && (long long)((N + 63) / 64) * mb >= 128) return 812;
    return (long long)((N + 31) / 32) * mb <= 256 ? 811 : 0;
  }
  auto fills = [&](int bn) {
    const long long blocks = (long long)((N + bn - 1) / bn) * ((M + 255) / 256);
    const long long rounds = (blocks + 255) / 256;
    return blocks >= 256 && blocks * 10 >= rounds * 256 * 9;
  };
  if (paired) return fills(64) ? 821 : 0;
  return fills(128) ? 822 : fills(192) ? 823 : 0;
}

// The wide instances in the code object (their staging fits 160 KB of LDS).
bool wide_instance(int tile, int bits, bool paired) {
  if (paired) return tile == 241;
  return bits == 4 || tile == 241 || tile == 242 || tile == 441;
}

// From this many rows (and K % 256 == 0: every group size up to 128 then gives an
// even number of groups per row) the automatic plan takes the wide-tile kernels.
constexpr int kWideRows = 512;

bool wide_auto_rows(int M, int K) { return M >= kWideRows && K % 256 == 0; }

// The automatic wide plan. Tiles: q/k/v-like outputs that fill the chip with
// 384-column blocks take 128 x 96 waves (243), other grids of >= 224 blocks of 128 x
// 256 take 8-wave blocks of 128 x 32 waves (441), smaller ones 128 x 32 waves in
// 4-wave blocks (241), split along k when fewer than 160 blocks would run. The
// paired gate/up always takes 241 (two accumulator sets). Measured on MI355X for
// the Llama-3-8B projections at 2048 rows (us, o / down / q/k/v): 242 84.8 / 253.5 /
// 145.7, 441 83.4 / 253.9 / 139.8, 243 - / - / 114.3; at 512 rows 241 with the split
// rule: q/k/v 38.7, o 32.9, gate/up 134.6, down 78.6. The choice does not depend on
// the code width (243 has no 8-bit instance; the launch substitutes 441, whose grid
// is then unsplit too), so the workspace queries, which do not know it, agree.
void wide_auto_plan(int M, int N, int K, bool paired, int* tile, int* splits) {
  const long long mb = (M + 127) / 128;
  auto blocks = [&](int bn) { return (long long)((N + bn - 1) / bn) * mb; };
  int t = 241;
  if (!paired && N % 384 == 0 && blocks(384) >= 224)
    t = 243;
  else if (!paired && blocks(256) >= 224)
    t = 441;
  const long long b = t == 243 ? blocks(384) : t == 441 ? blocks(256) : blocks(128);
  int s = 1;
  if (b < 160) s = (int)((256 + b - 1) / b);
  const int most = (K / 128) / 2;  // at least two 128-k steps per slice
  if (s > most) s = most > 1 ? most : 1;
  *tile = t;
  *splits = s;
}

// Automatic codes (tile = splits = 0) resolved to explicit ones for long prompts;
// other codes pass unchanged (the 16x16 kernel's own plan handles tile = 0 below
// kWideRows).
void resolve_auto(int M, int N, int K, bool paired, int* tile, int* splits) {
  if (*tile == 0 && *splits == 0 && wide_auto_rows(M, K)) wide_auto_plan(M, N, K, paired, tile, splits);
}

GemmPlan gemm_plan(int M, int N, int K, int tile, int splits, bool paired) {
  GemmPlan p{};
  if (lds_code(tile)) {
    p.lds = true;
    p.lds_bm = tile / 10 == 82 ? 256 : 128;
    p.lds_waves = tile / 10 == 82 ? 8 : 4;
    p.lds_bn = tile == 811 || tile == 813 ? 32 : tile == 823 ? 192 : tile == 822 ? 128 : 64;
    p.splits = 1;
    p.kslice = K;
    if (lds_split_code(tile)) {
      // k slices of whole 64-k steps; automatic: ~232 blocks (232 / column blocks,
      // rounded), at least two steps a slice
      const int steps = K / 64;
      int s = splits;
      if (s <= 0) {
        const long long cols = (long long)((N + p.lds_bn - 1) / p.lds_bn) * ((M + 127) / 128);
        s = (int)((232 + cols / 2) / cols);
        if (s > steps / 2) s = steps / 2;
      }
      if (s < 1) s = 1;
      if (s > steps) s = steps;
      p.kslice = ((steps + s - 1) / s) * 64;
      p.splits = (K + p.kslice - 1) / p.kslice;
    }
    return p;
  }
  if (wide_code(tile)) {
    p.wide_nw = 2 * (tile / 100);
    p.wide_mt = (tile / 10) % 10;
    p.wide_nt = tile % 10;
  } else if (tile == 0) {
    // Up to M = 128 (the latency-bound prefill of a small model wants blocks)
    // 32-row blocks - a wave's dequant per k-step does not depend on the rows,
    // so halving them halves its MFMA time and doubles the blocks (Qwen2-0.5B at
    // 128 rows: o + reduce/norm 8.6 -> 7.9 us, down 13.1 -> 12.4, prefill 104.0k
    // -> 106.1k tok/s) - except the paired gate/up, faster on 64-row blocks
    // (11.3 against 12.3 us); 128-row blocks beyond: measured on MI355X with the
    // 128-k step kernel, M = 256: gate/up 114 -> 83 us, down 84 -> 58 us.
    p.tm = M <= 128 ? (paired ? 4 : 2) : 8;
    const long long mb = (M + 16 * p.tm - 1) / (16 * p.tm);
    // 128-column blocks with 128-row blocks, except for the paired gate/up,
    // whose two accumulator sets fit one wave's registers only at 64 columns
    // (Llama-8B shapes, gate/up at M = 512 / 2048: 161 / 571 us at 64 columns,
    // 183 / 638 at 128).
    p.tn = !paired && (p.tm == 8 || mb * ((N + 127) / 128) >= 256) ? 2 : 1;
  } else {
    p.tn = tile / 10;
    p.tm = tile % 10;
  }
  const long long tiles = (long long)((N + p.bn() - 1) / p.bn()) * ((M + p.bm() - 1) / p.bm());
  const int ksteps = (K + 127) / 128;  // the kernel's k-steps (the last may be half)
  int s = splits;
  if (s <= 0) {
    // Split the reduction of small grids: up to 256 rows, to ~256 blocks when
    // there are fewer than 128 tiles; beyond, to ~512 blocks when there are
    // fewer than 256 (Llama-8B at 512 tokens: o 100.6 -> 50.8 us, down 340 ->
    // 136 us; 448 tiles or more run fastest unsplit).
    const long long few = M <= 256 ? 128 : 256, target = M <= 256 ? 256 : 512;
    s = 1;
    if (tiles < few) {
      s = (int)((target + tiles - 1) / tiles);
      if (s < 1) s = 1;
    }
  }
  if (s > ksteps) s = ksteps;
  const int steps_per = (ksteps + s - 1) / s;
  p.kslice = steps_per * 128;
  p.splits = (K + p.kslice - 1) / p.kslice;
  return p;
}

}  // namespace

// Automatic codes resolved to the explicit plan aoto_hip_w4_gemm would run (for
// the allocation-free entry point, which sizes its split against its scratch).
extern "C++" void aoto::resolve_gemm_codes(int M, int N, int K, int group, bool gate, int* tile, int* splits) {
  if (*tile == 0 && *splits == 0) {
    if (const int code = lds_auto(4, M, N, K, group, false, gate, false)) {
      *tile = code;
      *splits = gemm_plan(M, N, K, code, 0, false).splits;  // 1 unless the short split form
      return;
    }
  }
  resolve_auto(M, N, K, false, tile, splits);
}

namespace {

// The q/k/v projection's plan: the requested tile and split count, or with 0 the
// unsplit plan when its blocks' columns are whole heads (the RoPE epilogue: one
// launch, measured on MI355X at M = 128 / 512 / 2048: 9.9 / 61.5 / 142.6 us against
// 9.8 / 63.6 / 148.7 for the auto split and its RoPE reduce), on 32-row blocks up to
// 128 rows (twice the blocks; each wave's dequant per step is the same: 7.5 against
// 9.3 us on 64-row blocks for Qwen2-0.5B at 128 rows), else the auto split.
void qkv_rope_plan(int M, int N, int K, int head_dim, int* tile, int* splits) {
  if (*splits != 0 || head_dim <= 0 || wide_code(*tile) || lds_code(*tile)) return;
  const int t = *tile == 0 && M <= 128 && 64 % head_dim == 0 ? 12 : *tile;
  const GemmPlan p = gemm_plan(M, N, K, t, 1, false);
  const int bn = 64 * p.tn;
  if (bn % head_dim == 0 && N % bn == 0) {
    *tile = t;
    *splits = 1;
  }
}

}  // namespace

size_t aoto_hip_w4_gemm_workspace(int M, int N, int K, int tile, int splits) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return 0;
  // automatic codes: enough for the short prompts' split dequant-once plan too, which
  // the group, code width and epilogue (not known here) may select
  const int short_split = tile == 0 && splits == 0 ? lds_short_single(M, N, K) : 0;
  resolve_auto(M, N, K, false, &tile, &splits);
  const GemmPlan p = gemm_plan(M, N, K, tile, splits, false);
  size_t bytes = p.splits > 1 || lds_split_code(tile) ? (size_t)p.splits * M * N * sizeof(float) : 0;
  if (short_split) {
    const size_t lds_bytes = (size_t)gemm_plan(M, N, K, short_split, 0, false).splits * M * N * sizeof(float);
    if (lds_bytes > bytes) bytes = lds_bytes;
  }
  return bytes;
}

size_t aoto_hip_w4_gemm_gate_up_workspace(int M, int N, int K, int tile, int splits) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return 0;
  resolve_auto(M, N, K, true, &tile, &splits);
  const GemmPlan p = gemm_plan(M, N, K, tile, splits, true);
  return p.splits > 1 ? 2 * (size_t)p.splits * M * N * sizeof(float) : 0;
}

size_t aoto_hip_w4_gemm_qkv_rope_workspace(int M, int K, int tile, int splits, int query_heads, int kv_heads,
                                           int head_dim) {
  if (query_heads <= 0 || kv_heads <= 0 || head_dim <= 0) return 0;
  const int N = (query_heads + 2 * kv_heads) * head_dim;
  if (!wide_auto_rows(M, K)) qkv_rope_plan(M, N, K, head_dim, &tile, &splits);
  return aoto_hip_w4_gemm_workspace(M, N, K, tile, splits);
}

}  // extern "C"

namespace {

// The unsplit GEMM's tail for the q/k/v projection: RoPE of q/k, q head-major and
// the K/V cache fill from y (the GEMM's output with its bias).
// (aoto_rope_qkv_rows: one thread per 4 + 4 partner columns, 8-byte accesses)
int rope_after_gemm(const void* y, int M, const aoto::QkvRope& rope, void* stream) {
  const int D = rope.head_dim;
  long long items = (long long)M * (rope.query_heads + 2 * rope.kv_heads) * (D / 8);
  if (rope.zero_prefix) items += 2LL * rope.kv_heads * rope.slot0 * D / 4;
  return launch("aoto_rope_qkv_rows", dim3(blocks_for(items, 256)), dim3(256), 0, stream, y, M, rope.positions,
                rope.cos_table, rope.sin_table, rope.q_out, rope.pair, rope.query_heads, rope.kv_heads, D, rope.cap,
                rope.slot0, rope.zero_prefix);
}

// The prefill GEMM of either code width (the kernels differ only in how many
// packed words make one lane's 8-code operand).
// With up_words / up_scales (the gate/up entry points) the launch is the paired
// form: `words` is the gate projection, y = bf16(up * silu(bf16(gate))).
int packed_gemm(int bits, const void* x, const int32_t* words, const void* scales, const void* bias,
                const void* residual, const void* gate, void* y, int M, int N, int K, int group, int tile,
                int splits, void* workspace, void* stream, const int32_t* up_words = nullptr,
                const void* up_scales = nullptr, const void* norm_weight = nullptr, float eps = 0.f,
                void* norm_out = nullptr, const aoto::QkvRope* rope = nullptr) {
  const bool paired = up_words != nullptr;
  const char* what = paired ? (bits == 4 ? "w4_gemm_gate_up" : "w8_gemm_gate_up") : (bits == 4 ? "w4_gemm" : "w8_gemm");
  if (!x || !words || !scales || !y || (paired && !up_scales))
    return fail(AOTO_ERR_ARGUMENT, "%s: null pointer", what);
  if (paired && (bias || residual || gate)) return fail(AOTO_ERR_ARGUMENT, "%s: no other epilogue", what);
  if (M <= 0 || N <= 0 || K <= 0)
    return fail(AOTO_ERR_ARGUMENT, "%s: empty shape M=%d N=%d K=%d", what, M, N, K);
  if (K % 64 != 0 || N % 16 != 0 || group <= 0 || group % 32 != 0 || K % group != 0)
    return fail(AOTO_ERR_UNSUPPORTED, "%s: needs K %% 64 == 0, N %% 16 == 0, group %% 32 == 0 dividing K "
                "(M=%d N=%d K=%d group=%d)", what, M, N, K, group);
  const int epilogues = (bias != nullptr) + (residual != nullptr) + (gate != nullptr);
  if (epilogues > 1) return fail(AOTO_ERR_ARGUMENT, "%s: at most one of bias, residual, gate", what);
  if (!aligned16(x) || !aligned8(y) || (bias && !aligned8(bias)) || (residual && !aligned8(residual)) ||
      (gate && !aligned8(gate)) || !aligned16(words) || (paired && !aligned16(up_words)))
    return fail(AOTO_ERR_ARGUMENT, "%s: x and words must be 16-byte aligned, y/bias/residual/gate 8-byte aligned",
                what);
  if (tile != 0 && tile != 12 && tile != 14 && tile != 18 && tile != 24 && tile != 28 && !wide_code(tile) &&
      !lds_code(tile))
    return fail(AOTO_ERR_ARGUMENT, "%s: tile code %d is not one of 12, 14, 18, 24, 28, 241, 242, 243, 281, 441, "
                "811, 812, 813, 814, 821, 822, 823", what, tile);
  if (lds_code(tile)) {
    if (bits != 4 || lds_paired_code(tile) != paired || gate != nullptr || (splits > 1 && !lds_split_code(tile)))
      return fail(AOTO_ERR_ARGUMENT, "%s: tile %d is the unsplit 4-bit %s form without a gate epilogue", what, tile,
                  lds_paired_code(tile) ? "paired" : "single");
    if ((group & (group - 1)) != 0 || K % 64 != 0 || (K / group) % 2 != 0)
      return fail(AOTO_ERR_UNSUPPORTED, "%s: tile %d needs K %% 64 == 0 and an even number of power-of-two groups "
                  "per row (K=%d group=%d)", what, tile, K, group);
    // the kernel's per-lane load offsets are 32-bit
    if ((long long)M * K * 2 >= (1LL << 31) || (long long)N * K / 2 >= (1LL << 31))
      return fail(AOTO_ERR_UNSUPPORTED, "%s: tile %d needs X and the packed words under 2 GiB (M=%d N=%d K=%d)", what,
                  tile, M, N, K);
  }
  if (wide_code(tile)) {
    if (!wide_instance(tile, bits, paired))
      return fail(AOTO_ERR_ARGUMENT, "%s: no wide tile %d instance for %d-bit%s codes", what, tile, bits,
                  paired ? " paired" : "");
    if ((group & (group - 1)) != 0 || K % 128 != 0 || (K / group) % 2 != 0)
      return fail(AOTO_ERR_UNSUPPORTED, "%s: wide tile %d needs K %% 128 == 0 and an even number of "
                  "power-of-two groups per row (K=%d group=%d)", what, tile, K, group);
  }
  if (tile == 0 && splits == 0) {
    if (const int code = lds_auto(bits, M, N, K, group, paired, gate != nullptr, rope != nullptr)) tile = code;
  }
  resolve_auto(M, N, K, paired, &tile, &splits);
  if (bits == 8 && tile == 243) tile = 441;  // no 8-bit 243 instance; the same (unsplit) grid class
  const GemmPlan p = gemm_plan(M, N, K, tile, splits, paired);
  const bool lds_split = lds_split_code(tile);  // partials at every split count, 1 included
  if ((p.splits > 1 || lds_split) && (workspace == nullptr || !aligned16(workspace)))
    return fail(AOTO_ERR_ARGUMENT, "%s: %d-way split-K needs a 16-byte aligned workspace of "
                "aoto_hip_w4_gemm%s_workspace() bytes", what, p.splits, paired ? "_gate_up" : "");
  const int bn = p.bn(), bm = p.bm();
  const bool split = p.splits > 1 || lds_split;
  const bool wide = p.wide_mt != 0;
  char family[24];
  if (wide)
    snprintf(family, sizeof(family), "w%dx%dx%d", p.wide_mt, p.wide_nt, p.wide_nw);
  else
    snprintf(family, sizeof(family), "n%d_m%d", p.tn, p.tm);
  const dim3 grid((N + bn - 1) / bn, (M + bm - 1) / bm, p.splits);
  float* partials = split ? static_cast<float*>(workspace) : nullptr;
  const long long quads = (long long)M * N / 4;
  char name[64];
  if (lds_split) {
    // dequant-once split partials; the reduce launches below sum them with the epilogue
    snprintf(name, sizeof(name), "aoto_w4_gemm_d4c%dw%dx1_split", p.lds_bn / 32, p.lds_bn / 32);
    if (int st = launch(name, grid, dim3(p.threads()), 0, stream, x, words, scales, partials, M, N, K, group,
                        p.kslice))
      return st;
  } else if (p.lds) {
    // dequant-once kernel: unsplit, its own epilogues; norm / RoPE launches follow as
    // after any unsplit GEMM
    int st;
    if (paired) {
      const char* kernel = p.lds_bm == 256 ? "aoto_w4_gemm_d8w2x1_paired"
                           : p.lds_bn == 64 ? "aoto_w4_gemm_d4w2x1_paired"
                                            : "aoto_w4_gemm_d4c1w1x1_paired";
      st = launch(kernel, grid, dim3(p.threads()), 0, stream, x, words, scales, up_words, up_scales, y, M, N, K,
                  group);
    } else {
      snprintf(name, sizeof(name), "aoto_w4_gemm_d8w2x%d_b%d_r%d", p.lds_bn / 64, bias != nullptr,
               residual != nullptr);
      st = launch(name, grid, dim3(p.threads()), 0, stream, x, words, scales, bias, residual, y, M, N, K, group);
    }
    if (st || paired) return st;
    if (norm_out != nullptr)
      return launch("aoto_rms_norm", dim3((M + 3) / 4), dim3(256), 0, stream, y, norm_weight, eps, norm_out, M, N);
    if (rope != nullptr) return rope_after_gemm(y, M, *rope, stream);
    return AOTO_OK;
  }
  if (paired) {
    snprintf(name, sizeof(name), "aoto_w%d_gemm_%s_paired", bits, family);
    if (int st = launch(name, grid, dim3(p.threads()), 0, stream, x, words, scales, up_words, up_scales, y, M, N, K, group,
                        p.kslice, partials))
      return st;
    if (!split) return AOTO_OK;
    return launch("aoto_w4_gemm_reduce_paired", dim3(blocks_for(quads, 256)), dim3(256), 0, stream,
                  (const float*)partials, p.splits, y, M, N);
  }
  if (rope != nullptr && !split && !wide && bn % rope->head_dim == 0 && N % bn == 0) {
    // unsplit with whole heads per block: bias, RoPE and the cache fill in the epilogue
    snprintf(name, sizeof(name), "aoto_w%d_gemm_n%d_m%d_rope_b%d", bits, p.tn, p.tm, bias != nullptr);
    return launch(name, grid, dim3(256), 0, stream, x, words, scales, bias, y, M, N, K, group, *rope);
  }
  if (!lds_split) {
    const int b = !split && bias != nullptr, r = !split && residual != nullptr, g = !split && gate != nullptr;
    snprintf(name, sizeof(name), "aoto_w%d_gemm_%s_b%d_r%d_g%d", bits, family, b, r, g);
    if (int st = launch(name, grid, dim3(p.threads()), 0, stream, x, words, scales, bias, residual, gate, y, M, N, K,
                        group, p.kslice, partials))
      return st;
  }
  if (norm_out != nullptr) {
    if (!split)
      return launch("aoto_rms_norm", dim3((M + 3) / 4), dim3(256), 0, stream, y, norm_weight, eps, norm_out, M, N);
    return launch("aoto_w4_gemm_reduce_norm", dim3(M), dim3(256), 0, stream, (const float*)partials,
                  p.splits, residual, y, norm_weight, eps, norm_out, M, N);
  }
  if (rope != nullptr) {
    // q/k/v: unsplit, the GEMM stored y with its bias and the RoPE / cache fill
    // kernel follows; split, the sum, bias, RoPE and cache fill are one launch
    if (!split) return rope_after_gemm(y, M, *rope, stream);
    const int D = rope->head_dim;
    long long items = (long long)M * (N / D) * (D / 8);
    if (rope->zero_prefix) items += 2LL * rope->kv_heads * rope->slot0 * D / 4;
    return launch("aoto_w4_gemm_reduce_rope", dim3(blocks_for(items, 256)), dim3(256), 0, stream,
                  (const float*)partials, p.splits, bias, y, M, rope->positions, rope->cos_table, rope->sin_table,
                  rope->q_out, rope->pair, rope->query_heads, rope->kv_heads, D, rope->cap, rope->slot0,
                  rope->zero_prefix);
  }
  if (!split) return AOTO_OK;
  return launch("aoto_w4_gemm_reduce", dim3(blocks_for(quads, 256)), dim3(256), 0, stream,
                (const float*)partials, p.splits, bias, residual, gate, y, M, N);
}


// The packed q/k/v projection (+ bias) with its RoPE and the layer's cache fill.
int qkv_rope_gemm(int bits, const void* x, const int32_t* words, const void* scales, const void* bias, void* y,
                  int M, int K, int group, int tile, int splits, void* workspace, const int64_t* positions,
                  const void* cos_table, const void* sin_table, void* q_out, void* pair, int query_heads,
                  int kv_heads, int head_dim, int capacity, int slot0, int zero_prefix, void* stream) {
  const char* what = bits == 4 ? "w4_gemm_qkv_rope" : "w8_gemm_qkv_rope";
  if (!positions || !cos_table || !sin_table || !q_out || !pair) return fail(AOTO_ERR_ARGUMENT, "%s: null pointer", what);
  if (query_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || head_dim % 8 != 0)
    return fail(AOTO_ERR_ARGUMENT, "%s: bad heads (Hq=%d Hkv=%d D=%d)", what, query_heads, kv_heads, head_dim);
  if (M <= 0 || slot0 < 0 || slot0 + M > capacity)
    return fail(AOTO_ERR_ARGUMENT, "%s: slots [%d, %d) exceed capacity %d", what, slot0, slot0 + M, capacity);
  if (!aligned8(q_out) || !aligned8(pair) || !aligned8(cos_table) || !aligned8(sin_table) || (bias && !aligned8(bias)))
    return fail(AOTO_ERR_ARGUMENT, "%s: q_out, pair, tables and bias must be 8-byte aligned", what);
  if (y == q_out || y == pair || y == x) return fail(AOTO_ERR_ARGUMENT, "%s: y must not alias x, q_out or pair", what);
  const aoto::QkvRope rope{(const long long*)positions, (const uint16_t*)cos_table, (const uint16_t*)sin_table,
                           (uint16_t*)q_out, (uint16_t*)pair, query_heads, kv_heads, head_dim, capacity, slot0,
                           zero_prefix};
  const int N = (query_heads + 2 * kv_heads) * head_dim;
  if (!wide_auto_rows(M, K)) qkv_rope_plan(M, N, K, head_dim, &tile, &splits);
  return packed_gemm(bits, x, words, scales, bias, nullptr, nullptr, y, M, N, K, group, tile, splits, workspace,
                     stream, nullptr, nullptr, nullptr, 0.f, nullptr, &rope);
}

// GEMM with a residual epilogue followed by the row RMSNorm of its result.
int residual_norm_gemm(int bits, const void* x, const int32_t* words, const void* scales, const void* residual,
                       void* y, int M, int N, int K, int group, int tile, int splits, void* workspace,
                       const void* norm_weight, float eps, void* norm_out, void* stream) {
  const char* what = bits == 4 ? "w4_gemm_residual_norm" : "w8_gemm_residual_norm";
  if (!residual || !norm_weight || !norm_out) return fail(AOTO_ERR_ARGUMENT, "%s: null pointer", what);
  if (N % 8 != 0 || N > 4096)
    return fail(AOTO_ERR_UNSUPPORTED, "%s: the norm takes rows of N %% 8 == 0 up to 4096 (N=%d)", what, N);
  if (!aligned16(y) || !aligned16(residual) || !aligned16(norm_weight) || !aligned16(norm_out))
    return fail(AOTO_ERR_ARGUMENT, "%s: y, residual, norm weight and norm output must be 16-byte aligned", what);
  if (norm_out == y || norm_out == residual || norm_out == x)
    return fail(AOTO_ERR_ARGUMENT, "%s: the norm output must not alias x, y or the residual", what);
  return packed_gemm(bits, x, words, scales, nullptr, residual, nullptr, y, M, N, K, group, tile, splits, workspace,
                     stream, nullptr, nullptr, norm_weight, eps, norm_out);
}

}  // namespace

extern "C" {

int aoto_hip_w4_gemm(const void* x, const int32_t* words, const void* scales, const void* bias,
                     const void* residual, const void* gate, void* y, int M, int N, int K, int group,
                     int tile, int splits, void* workspace, void* stream) {
  return packed_gemm(4, x, words, scales, bias, residual, gate, y, M, N, K, group, tile, splits, workspace,
                     stream);
}

int aoto_hip_w8_gemm(const void* x, const int32_t* words, const void* scales, const void* bias,
                     const void* residual, const void* gate, void* y, int M, int N, int K, int group,
                     int tile, int splits, void* workspace, void* stream) {
  return packed_gemm(8, x, words, scales, bias, residual, gate, y, M, N, K, group, tile, splits, workspace,
                     stream);
}

int aoto_hip_w4_gemm_gate_up(const void* x, const int32_t* gate_words, const void* gate_scales,
                             const int32_t* up_words, const void* up_scales, void* y, int M, int N, int K,
                             int group, int tile, int splits, void* workspace, void* stream) {
  if (!up_words) return fail(AOTO_ERR_ARGUMENT, "w4_gemm_gate_up: null pointer");
  return packed_gemm(4, x, gate_words, gate_scales, nullptr, nullptr, nullptr, y, M, N, K, group, tile, splits,
                     workspace, stream, up_words, up_scales);
}

int aoto_hip_w8_gemm_gate_up(const void* x, const int32_t* gate_words, const void* gate_scales,
                             const int32_t* up_words, const void* up_scales, void* y, int M, int N, int K,
                             int group, int tile, int splits, void* workspace, void* stream) {
  if (!up_words) return fail(AOTO_ERR_ARGUMENT, "w8_gemm_gate_up: null pointer");
  return packed_gemm(8, x, gate_words, gate_scales, nullptr, nullptr, nullptr, y, M, N, K, group, tile, splits,
                     workspace, stream, up_words, up_scales);
}

int aoto_hip_w4_gemm_residual_norm(const void* x, const int32_t* words, const void* scales, const void* residual,
                                   void* y, int M, int N, int K, int group, int tile, int splits, void* workspace,
                                   const void* norm_weight, float eps, void* norm_out, void* stream) {
  return residual_norm_gemm(4, x, words, scales, residual, y, M, N, K, group, tile, splits, workspace,
                            norm_weight, eps, norm_out, stream);
}

int aoto_hip_w8_gemm_residual_norm(const void* x, const int32_t* words, const void* scales, const void* residual,
                                   void* y, int M, int N, int K, int group, int tile, int splits, void* workspace,
                                   const void* norm_weight, float eps, void* norm_out, void* stream) {
  return residual_norm_gemm(8, x, words, scales, residual, y, M, N, K, group, tile, splits, workspace,
                            norm_weight, eps, norm_out, stream);
}

int aoto_hip_w4_gemm_qkv_rope(const void* x, const int32_t* words, const void* scales, const void* bias, void* y,
                              int M, int K, int group, int tile, int splits, void* workspace, const int64_t* positions,
                              const void* cos_table, const void* sin_table, void* q_out, void* pair, int query_heads,
                              int kv_heads, int head_dim, int capacity, int slot0, int zero_prefix, void* stream) {
  return qkv_rope_gemm(4, x, words, scales, bias, y, M, K, group, tile, splits, workspace, positions, cos_table,
                       sin_table, q_out, pair, query_heads, kv_heads, head_dim, capacity, slot0, zero_prefix, stream);
}

int aoto_hip_w8_gemm_qkv_rope(const void* x, const int32_t* words, const void* scales, const void* bias, void* y,
                              int M, int K, int group, int tile, int splits, void* workspace, const int64_t* positions,
                              const void* cos_table, const void* sin_table, void* q_out, void* pair, int query_heads,
                              int kv_heads, int head_dim, int capacity, int slot0, int zero_prefix, void* stream) {
  return qkv_rope_gemm(8, x, words, scales, bias, y, M, K, group, tile, splits, workspace, positions, cos_table,
                       sin_table, q_out, pair, query_heads, kv_heads, head_dim, capacity, slot0, zero_prefix, stream);
}

int aoto_hip_w8_quantize(const void* weight, int weight_is_f32, int rows, int inner, int group,
                         int32_t* packed, void* scales_bf16, float* scales_f32, void* stream) {
  if (!weight || !packed || !scales_bf16) return fail(AOTO_ERR_ARGUMENT, "w8_quantize: null pointer");
  if (rows <= 0 || inner <= 0) return fail(AOTO_ERR_ARGUMENT, "w8_quantize: empty shape %dx%d", rows, inner);
  if (group <= 0 || group % 4 != 0 || inner % group != 0)
    return fail(AOTO_ERR_ARGUMENT, "w8_quantize: group %d must be a positive multiple of 4 dividing %d",
                group, inner);
  const long long tasks = (long long)rows * (inner / group);
  return launch("aoto_w8_quantize", dim3(blocks_for(tasks, 256)), dim3(256), 0, stream, weight, weight_is_f32,
                rows, inner, group, packed, scales_bf16, scales_f32);
}

int aoto_hip_w8_dequantize(const int32_t* packed, const void* scales, int rows, int inner, int group,
                           void* out, void* stream) {
  if (!packed || !scales || !out) return fail(AOTO_ERR_ARGUMENT, "w8_dequantize: null pointer");
  if (rows <= 0 || inner <= 0 || inner % 4 != 0)
    return fail(AOTO_ERR_ARGUMENT, "w8_dequantize: bad shape %dx%d", rows, inner);
  if (group <= 0 || group % 4 != 0 || inner % group != 0)
    return fail(AOTO_ERR_ARGUMENT, "w8_dequantize: bad group %d for inner %d", group, inner);
  if (!aligned8(out)) return fail(AOTO_ERR_ARGUMENT, "w8_dequantize: output must be 8-byte aligned");
  const long long words = (long long)rows * (inner / 4);
  return launch("aoto_w8_dequantize", dim3(blocks_for(words, 256)), dim3(256), 0, stream, packed, scales, rows,
                inner, group, out);
}

int aoto_hip_w8_gemv(const void* x, const int32_t* words, const void* scales, const int32_t* up_words,
                     const void* up_scales, const void* norm_weight, float eps, const void* bias, float alpha,
                     float beta, void* y, int K, int N, int group, void* stream) {
  if (!x || !words || !scales || !y) return fail(AOTO_ERR_ARGUMENT, "w8_gemv: null pointer");
  if ((up_words == nullptr) != (up_scales == nullptr))
    return fail(AOTO_ERR_ARGUMENT, "w8_gemv: paired projection needs both up_words and up_scales");
  const bool paired = up_words != nullptr;
  if (paired && bias != nullptr) return fail(AOTO_ERR_ARGUMENT, "w8_gemv: the paired epilogue takes no bias");
  if (N <= 0 || K <= 0) return fail(AOTO_ERR_ARGUMENT, "w8_gemv: empty shape K=%d N=%d", K, N);
  if (K % 16 != 0 || group <= 0 || group % 16 != 0 || K % group != 0 || K > 32768)
    return fail(AOTO_ERR_UNSUPPORTED, "w8_gemv: needs K %% 16 == 0, group %% 16 == 0 dividing K, K <= 32768 "
                "(K=%d group=%d)", K, group);
  if (!aligned16(x) || !aligned16(words) || (up_words && !aligned16(up_words)) ||
      (norm_weight && !aligned16(norm_weight)))
    return fail(AOTO_ERR_ARGUMENT, "w8_gemv: x, words and norm weight must be 16-byte aligned");
  // A wave holds R rows x U chunks of 16 codes per lane in flight: U covers the
  // row's chunks in one pass where it can (up to 4), R fills the rest of 4.
  const int chunks = K / 16;
  const int u = chunks <= 64 ? 1 : (chunks <= 128 ? 2 : 4);
  const int r = 4 / u;
  const int waves_needed = (N + r - 1) / r;
  const long long blocks_needed = (waves_needed + 3) / 4;
  const long long cap = (long long)cu_count() * 4;
  const unsigned blocks = (unsigned)(blocks_needed < cap ? blocks_needed : cap);
  const unsigned shared = (unsigned)(chunks * 32 + chunks * 4);
  char name[64];
  snprintf(name, sizeof(name), "aoto_w8_gemv_r%du%d_n%d_p%d_b%d", r, u, norm_weight != nullptr ? 1 : 0,
           paired ? 1 : 0, bias != nullptr ? 1 : 0);
  return launch(name, dim3(blocks), dim3(256), shared, stream, x, words, scales, up_words, up_scales,
                norm_weight, eps, bias, alpha, beta, y, K, N, group);
}

int aoto_hip_rms_norm(const void* x, const void* weight, float eps, void* out, int rows, int hidden,
                      void* stream) {
  if (!x || !weight || !out) return fail(AOTO_ERR_ARGUMENT, "rms_norm: null pointer");
  if (rows <= 0 || hidden <= 0) return fail(AOTO_ERR_ARGUMENT, "rms_norm: empty shape %dx%d", rows, hidden);
  if (hidden % 8 != 0) return fail(AOTO_ERR_UNSUPPORTED, "rms_norm: hidden %d is not a multiple of 8", hidden);
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out))
    return fail(AOTO_ERR_ARGUMENT, "rms_norm: x, weight and out must be 16-byte aligned");
  return launch("aoto_rms_norm", dim3((rows + 3) / 4), dim3(256), 0, stream, x, weight, eps, out, rows, hidden);
}

int aoto_hip_rope(const void* x, const void* cos_table, const void* sin_table, const int64_t* positions,
                  int rows_per_position, int position_count, void* out, int64_t rows, int head_dim,
                  void* stream) {
  if (!x || !cos_table || !sin_table || !positions || !out) return fail(AOTO_ERR_ARGUMENT, "rope: null pointer");
  if (rows <= 0 || head_dim <= 0 || head_dim % 2 != 0 || rows_per_position <= 0 || position_count <= 0)
    return fail(AOTO_ERR_ARGUMENT, "rope: bad shape rows=%lld head_dim=%d", (long long)rows, head_dim);
  long long items = (long long)rows * head_dim;
  return launch("aoto_rope", dim3(blocks_for(items, 256)), dim3(256), 0, stream, x, cos_table, sin_table,
                positions, rows_per_position, position_count, out, (long long)rows, head_dim);
}

int aoto_hip_rope_qkv_prefill(const void* qkv, const int64_t* positions, const void* cos_table,
                              const void* sin_table, void* q_out, void* pair, int batch, int tokens,
                              int query_heads, int kv_heads, int head_dim, int capacity, int slot0,
                              int zero_prefix, void* stream) {
  if (!qkv || !positions || !cos_table || !sin_table || !q_out || !pair)
    return fail(AOTO_ERR_ARGUMENT, "rope_qkv_prefill: null pointer");
  if (batch <= 0 || tokens <= 0 || query_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || head_dim % 2)
    return fail(AOTO_ERR_ARGUMENT, "rope_qkv_prefill: bad shape");
  if (slot0 < 0 || slot0 + tokens > capacity)
    return fail(AOTO_ERR_ARGUMENT, "rope_qkv_prefill: slots [%d, %d) exceed capacity %d", slot0, slot0 + tokens,
                capacity);
  long long items = (long long)batch * (query_heads + 2 * kv_heads) * tokens * head_dim;
  if (zero_prefix) items += 2LL * batch * kv_heads * slot0 * head_dim;
  return launch("aoto_rope_qkv_prefill", dim3(blocks_for(items, 256)), dim3(256), 0, stream, qkv, positions,
                cos_table, sin_table, q_out, pair, batch, tokens, query_heads, kv_heads, head_dim, capacity, slot0,
                zero_prefix);
}

int aoto_hip_rope_kv_cache_append(const void* row, int row_width, const void* cos_table, const void* sin_table,
                                  int position, const void* pair_in, void* pair_out, void* q_out, int batch,
                                  int query_heads, int kv_heads, int capacity, int head_dim, int query_start,
                                  int key_start, int value_start, int mode, int slot,
                                  const int32_t* step_state, void* stream) {
  if (!row || !cos_table || !sin_table || !pair_out || !q_out)
    return fail(AOTO_ERR_ARGUMENT, "rope_kv_cache_append: null pointer");
  if (mode != 0 && mode != 1) return fail(AOTO_ERR_ARGUMENT, "rope_kv_cache_append: mode must be 0 or 1");
  if (mode == 0 && (pair_in == nullptr || pair_in == pair_out))
    return fail(AOTO_ERR_ARGUMENT, "rope_kv_cache_append: the roll needs a separate input window");
  if (batch <= 0 || query_heads <= 0 || kv_heads <= 0 || capacity <= 0 || head_dim <= 0 || head_dim % 8)
    return fail(AOTO_ERR_ARGUMENT, "rope_kv_cache_append: bad shape");
  if (step_state != nullptr && mode != 1)
    return fail(AOTO_ERR_ARGUMENT, "rope_kv_cache_append: device step state drives the ring mode only");
  if (step_state == nullptr && (position < 0 || position >= capacity))
    return fail(AOTO_ERR_ARGUMENT, "rope_kv_cache_append: position %d outside the %d-row table", position,
                capacity);
  if (step_state == nullptr && mode == 1 && (slot < 0 || slot >= capacity))
    return fail(AOTO_ERR_ARGUMENT, "rope_kv_cache_append: slot %d outside capacity %d", slot, capacity);
  if (query_start < 0 || key_start < 0 || value_start < 0 || query_start + query_heads * head_dim > row_width ||
      key_start + kv_heads * head_dim > row_width || value_start + kv_heads * head_dim > row_width)
    return fail(AOTO_ERR_ARGUMENT, "rope_kv_cache_append: q/k/v columns exceed the row width %d", row_width);
  if (mode == 0 && (!aligned16(pair_in) || !aligned16(pair_out)))
    return fail(AOTO_ERR_ARGUMENT, "rope_kv_cache_append: windows must be 16-byte aligned");
  long long items = (long long)batch * (query_heads + kv_heads) * head_dim;
  if (mode == 0) items += 2LL * batch * kv_heads * (capacity - 1) * (head_dim / 8);
  return launch("aoto_rope_kv_append", dim3(blocks_for(items, 256)), dim3(256), 0, stream, row, row_width,
                cos_table, sin_table, position, pair_in, pair_out, q_out, batch, query_heads, kv_heads, capacity,
                head_dim, query_start, key_start, value_start, mode, slot, step_state);
}

size_t aoto_hip_decode_attention_workspace(int batch, int query_heads, int kv_heads, int capacity, int head_dim,
                                           int splits) {
  int s = 0, c = 0;
  decode_split(head_dim, capacity, splits, (long long)batch * query_heads, &s, &c);
  return s > 1 ? (size_t)batch * query_heads * s * (head_dim + 2) * sizeof(float) : 0;
}

namespace {

// Shared checks and split choice of the two decode-attention entry points.
int decode_attention_plan(const char* what, int batch, int query_heads, int kv_heads, int capacity, int head_dim,
                          int splits, const void* workspace, int* s, int* chunk) {
  if (batch <= 0 || query_heads <= 0 || kv_heads <= 0 || capacity <= 0 || query_heads % kv_heads)
    return fail(AOTO_ERR_ARGUMENT, "%s: bad shape (Hq=%d Hkv=%d cap=%d)", what, query_heads, kv_heads, capacity);
  if (head_dim != 64 && head_dim != 128)
    return fail(AOTO_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128)", what, head_dim);
  decode_split(head_dim, capacity, splits, (long long)batch * query_heads, s, chunk);
  if (*s > 1024)
    return fail(AOTO_ERR_UNSUPPORTED, "%s: %d keys need %d splits, more than the merge takes (1024)", what,
                capacity, *s);
  if (*s > 1 && workspace == nullptr)
    return fail(AOTO_ERR_ARGUMENT, "%s: %d keys in %d splits need a workspace", what, capacity, *s);
  return AOTO_OK;
}

int launch_merge(int rows, int splits, int head_dim, void* workspace, void* out, void* stream) {
  return launch("aoto_decode_attention_merge", dim3(rows), dim3(128), 0, stream, (const float*)workspace, splits,
                head_dim, out);
}

}  // namespace

int aoto_hip_decode_attention(const void* q, const void* keys, const void* values, int64_t kv_batch_stride,
                              int64_t kv_head_stride, const uint8_t* mask, int mask_batch_stride, int valid,
                              int ring_offset, int batch, int query_heads, int kv_heads, int capacity,
                              int head_dim, float scale, int splits, void* workspace,
                              const int32_t* step_state, void* out, void* stream) {
  if (!q || !keys || !values || !out) return fail(AOTO_ERR_ARGUMENT, "decode_attention: null pointer");
  int s = 0, chunk = 0;
  if (int st = decode_attention_plan("decode_attention", batch, query_heads, kv_heads, capacity, head_dim, splits,
                                     workspace, &s, &chunk))
    return st;
  if (mask == nullptr && step_state == nullptr &&
      (valid < 0 || valid > capacity || ring_offset < 0 || ring_offset >= capacity))
    return fail(AOTO_ERR_ARGUMENT, "decode_attention: valid %d / ring offset %d outside capacity %d", valid,
                ring_offset, capacity);
  if (!aligned16(q) || !aligned16(keys) || !aligned16(values) || (kv_head_stride % 8) || (kv_batch_stride % 8))
    return fail(AOTO_ERR_ARGUMENT, "decode_attention: q/keys/values must be 16-byte aligned");
  char name[64];
  const AttnShape as = attention_shape(head_dim, chunk);
  snprintf(name, sizeof(name), "aoto_decode_attention_d%d_w%dj%d", head_dim, as.waves, as.loads);
  if (int st = launch(name, dim3(s, batch * query_heads), dim3(64 * as.waves), 0, stream, q, keys, values,
                      (long long)kv_batch_stride, (long long)kv_head_stride, mask, mask_batch_stride, valid,
                      ring_offset, capacity, query_heads, kv_heads, scale, chunk, (float*)workspace, step_state,
                      out))
    return st;
  return s > 1 ? launch_merge(batch * query_heads, s, head_dim, workspace, out, stream) : AOTO_OK;
}

int aoto_hip_decode_rope_attention(const void* row, int row_width, int query_start, int key_start,
                                   int value_start, const void* cos_table, const void* sin_table, void* keys,
                                   void* values, int64_t kv_batch_stride, int64_t kv_head_stride, int position,
                                   int slot, int valid, int ring_offset, int batch, int query_heads, int kv_heads,
                                   int capacity, int head_dim, float scale, int splits, void* workspace,
                                   const int32_t* step_state, const void* rope_rows, void* out, void* stream) {
  if (!row || !cos_table || !sin_table || !keys || !values || !out)
    return fail(AOTO_ERR_ARGUMENT, "decode_rope_attention: null pointer");
  int s = 0, chunk = 0;
  if (int st = decode_attention_plan("decode_rope_attention", batch, query_heads, kv_heads, capacity, head_dim,
                                     splits, workspace, &s, &chunk))
    return st;
  if (query_start < 0 || key_start < 0 || value_start < 0 || query_start + query_heads * head_dim > row_width ||
      key_start + kv_heads * head_dim > row_width || value_start + kv_heads * head_dim > row_width)
    return fail(AOTO_ERR_ARGUMENT, "decode_rope_attention: q/k/v columns exceed the row width %d", row_width);
  if (step_state == nullptr &&
      (position < 0 || position >= capacity || slot < 0 || slot >= capacity || valid < 0 || valid > capacity ||
       ring_offset < 0 || ring_offset >= capacity))
    return fail(AOTO_ERR_ARGUMENT, "decode_rope_attention: position %d / slot %d / valid %d / offset %d outside "
                "capacity %d", position, slot, valid, ring_offset, capacity);
  if (!aligned16(keys) || !aligned16(values) || (kv_head_stride % 8) || (kv_batch_stride % 8) ||
      !aligned16(row) || !aligned16(cos_table) || !aligned16(sin_table) || (row_width % 8) || (query_start % 8))
    return fail(AOTO_ERR_ARGUMENT, "decode_rope_attention: keys/values/row/tables must be 16-byte aligned, "
                "row width and query start multiples of 8");
  // the kernel takes these packed (decode.h): 16-bit heads, starts and width,
  // a 9-bit chunk with a 22-bit capacity, 31-bit strides
  if (query_heads >= 65536 || kv_heads >= 65536 || row_width >= 65536 || chunk >= 512 || capacity >= (1 << 22) ||
      kv_batch_stride >= (int64_t)1 << 31 || kv_head_stride >= (int64_t)1 << 31 || kv_batch_stride < 0 ||
      kv_head_stride < 0)
    return fail(AOTO_ERR_UNSUPPORTED, "decode_rope_attention: heads, row width < 65536, capacity < 2^22 and "
                "strides < 2^31 elements needed");
  char name[64];
  const AttnShape as = attention_shape(head_dim, chunk);
  snprintf(name, sizeof(name), "aoto_decode_rope_attention_d%d_w%dj%d", head_dim, as.waves, as.loads);
  const int heads = query_heads | (kv_heads << 16), starts_qk = query_start | (key_start << 16);
  const int start_v_width = value_start | (row_width << 16), chunk_cap = chunk | (capacity << 9);
  if (int st = launch(name, dim3(s, batch * query_heads), dim3(64 * as.waves), 0, stream, row, rope_rows, keys,
                      values, (int)kv_head_stride, (int)kv_batch_stride, heads, starts_qk, start_v_width, chunk_cap,
                      valid, ring_offset, position, slot, scale, (float*)workspace, step_state, cos_table, sin_table,
                      out))
    return st;
  return s > 1 ? launch_merge(batch * query_heads, s, head_dim, workspace, out, stream) : AOTO_OK;
}

int aoto_hip_step_advance(int32_t* step_state, int capacity, void* stream) {
  if (!step_state || capacity <= 0) return fail(AOTO_ERR_ARGUMENT, "step_advance: bad arguments");
  return launch("aoto_step_advance", dim3(1), dim3(64), 0, stream, step_state, capacity);
}

int aoto_hip_prefill_attention(const void* q, const void* keys, const void* values, int64_t kv_batch_stride,
                               int64_t kv_head_stride, const uint8_t* mask, int64_t mask_batch_stride, int causal,
                               int key_start, int batch, int tokens, int key_tokens, int query_heads,
                               int kv_heads, int head_dim, float scale, void* out, void* stream) {
  if (!q || !keys || !values || !out) return fail(AOTO_ERR_ARGUMENT, "prefill_attention: null pointer");
  if (batch <= 0 || tokens <= 0 || key_tokens <= 0 || query_heads <= 0 || kv_heads <= 0 ||
      query_heads % kv_heads)
    return fail(AOTO_ERR_ARGUMENT, "prefill_attention: bad shape");
  if (head_dim != 64 && head_dim != 128)
    return fail(AOTO_ERR_UNSUPPORTED, "prefill_attention: head_dim %d (64 or 128)", head_dim);
  if (!aligned16(q) || !aligned16(keys) || !aligned16(values) || !aligned8(out) || (kv_head_stride % 8) ||
      (kv_batch_stride % 8))
    return fail(AOTO_ERR_ARGUMENT, "prefill_attention: q/keys/values 16-byte, out 8-byte aligned");
  // one block per (128-query tile, batch, query head), the query tile slowest.
  // Grids that do not fill two 4-wave blocks per CU use 8-wave blocks whose two
  // wave groups split the keys (every CU then runs two waves per SIMD throughout).
  // A grid that fills at most a quarter (half) of the CUs - a short prompt:
  // Qwen2's 128 tokens make 14 blocks, Llama-3-8B's 512 make 128 - takes 32-query
  // (64-query) blocks of two 1-wave (2-wave) key groups instead: 4x (2x) the
  // blocks, one wave per SIMD (32-query blocks at D = 64 only).
  long long blocks = (long long)((tokens + 127) / 128) * batch * query_heads;
  if (blocks > 0x7FFFFFFFLL) return fail(AOTO_ERR_UNSUPPORTED, "prefill_attention: grid too large");
  const bool split_keys = blocks <= 2LL * cu_count();
  int queries = 128;  // per block
  if (mask == nullptr) {
    if (head_dim == 64) queries = 4 * blocks <= cu_count() ? 32 : 2 * blocks <= cu_count() ? 64 : 128;
    else if (2 * blocks <= cu_count()) queries = 64;  // D = 128 has no 32-query instance (registers)
  }
  if (queries < 128) blocks = (long long)((tokens + queries - 1) / queries) * batch * query_heads;
  char name[64];
  snprintf(name, sizeof(name), "aoto_flash_attention_d%d%s%s%s", head_dim, split_keys ? "_k2" : "", mask ? "_m" : "",
           queries == 32 ? "_q32" : queries == 64 ? "_q64" : "");
  const unsigned threads = queries < 128 ? 2 * 2 * queries : split_keys ? 512 : 256;
  return launch(name, dim3((unsigned)blocks), dim3(threads), 0, stream, q, keys,
                values,
                (long long)kv_batch_stride,
                (long long)kv_head_stride, mask, (long long)mask_batch_stride, causal, key_start, tokens,
                key_tokens, batch, query_heads, kv_heads, scale, out);
}

int aoto_hip_embedding(const void* weight, const int64_t* ids, int count, int hidden, int64_t vocab, void* out,
                       int* error, void* stream) {
  if (!weight || !ids || !out) return fail(AOTO_ERR_ARGUMENT, "embedding: null pointer");
  if (count <= 0 || hidden <= 0 || vocab <= 0) return fail(AOTO_ERR_ARGUMENT, "embedding: empty shape");
  if (hidden % 8 != 0) return fail(AOTO_ERR_UNSUPPORTED, "embedding: hidden %d is not a multiple of 8", hidden);
  if (!aligned16(weight) || !aligned16(out)) return fail(AOTO_ERR_ARGUMENT, "embedding: 16-byte alignment");
  long long items = (long long)count * (hidden / 8);
  return launch("aoto_embedding", dim3(blocks_for(items, 256)), dim3(256), 0, stream, weight, ids, count, hidden,
                (long long)vocab, out, error);
}

size_t aoto_hip_w4_gemv_argmax_keys(int K, int N, int group) {
  StreamShape ss{};
  if (N <= 0 || K <= 0 || !argmax_shape(K, N, group, &ss)) return 0;
  const StreamLaunch l = stream_launch(ss, K, N, group);
  return (size_t)(l.grid * l.wpb);
}

int aoto_hip_w4_gemv_argmax(const void* x, const int32_t* words, const void* scales, const void* norm_weight,
                            float eps, void* y, int K, int N, int group, uint64_t* keys, size_t key_count,
                            void* stream) {
  if (!x || !words || !scales || !y || !keys) return fail(AOTO_ERR_ARGUMENT, "w4_gemv_argmax: null pointer");
  if (N <= 0 || K <= 0) return fail(AOTO_ERR_ARGUMENT, "w4_gemv_argmax: empty shape K=%d N=%d", K, N);
  StreamShape ss{};
  if (!argmax_shape(K, N, group, &ss))
    return fail(AOTO_ERR_UNSUPPORTED, "w4_gemv_argmax: needs K %% 32 == 0, a power-of-two group >= 32 with an "
                "even number of groups per row, K <= 6144 (K=%d group=%d)", K, group);
  if (!aligned16(x) || !aligned16(words) || (norm_weight && !aligned16(norm_weight)) || !aligned4(scales) ||
      !aligned8(keys))
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv_argmax: x, words and norm weight must be 16-byte aligned, scales "
                "4-byte, keys 8-byte");
  // The K = 896 and K = 4096 LM heads with their final norm stage the
  // normalized x once per 4-wave block instead of once per wave
  // (aoto_w4_gemv_x8x4_n1_argmax: Qwen2's 151936 rows 14.87-14.94 -> 14.82-14.84
  // us; aoto_w4_gemv_x32x4_n1_argmax: Llama-3's 128256 rows 44.1-44.3 -> 43.4-43.5
  // us; same-box A/Bs). Only where the per-wave form already runs 4-wave blocks,
  // so the grid, and the key count aoto_hip_w4_gemv_argmax_keys reports, match.
  const bool blockx = norm_weight != nullptr && !ss.direct && ss.cpl == 4 && (ss.lpr == 8 || ss.lpr == 32) &&
                      stream_launch(ss, K, N, group).wpb == 4;
  if (blockx) ss.block_x = true;
  const StreamLaunch l = stream_launch(ss, K, N, group);
  if (key_count < (size_t)(l.grid * l.wpb))
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv_argmax: %zu keys given, %lld needed (aoto_hip_w4_gemv_argmax_keys)",
                key_count, l.grid * l.wpb);
  char sname[64];
  snprintf(sname, sizeof(sname), "aoto_w4_gemv_%s%dx%d_n%d_argmax", blockx ? "x" : "s", ss.lpr, ss.cpl,
           norm_weight ? 1 : 0);
  const void* none = nullptr;
  return launch(sname, dim3((unsigned)l.grid), dim3(64 * l.wpb), l.shared, stream, words, scales, x, norm_weight, K,
                N, l.shift, l.wpb, none, none, none, eps, 1.0f, 0.0f, y, keys);
}

int aoto_hip_argmax_finish(const uint64_t* keys, int key_count, int64_t* token_out, int64_t* history,
                           int* history_len, int32_t* step_state, int capacity, const void* embedding,
                           int64_t embedding_rows, int hidden, void* hidden_out, int* error,
                           const void* cos_table, const void* sin_table, int head_dim, void* rope_rows,
                           void* stream) {
  if (!keys || !token_out || key_count <= 0) return fail(AOTO_ERR_ARGUMENT, "argmax_finish: bad arguments");
  if ((history == nullptr) != (history_len == nullptr))
    return fail(AOTO_ERR_ARGUMENT, "argmax_finish: a token history needs both pointers");
  if (step_state && capacity <= 0) return fail(AOTO_ERR_ARGUMENT, "argmax_finish: step state needs a capacity");
  if (embedding && (!hidden_out || hidden <= 0 || hidden % 8 != 0 || embedding_rows <= 0 ||
                    !aligned16(embedding) || !aligned16(hidden_out)))
    return fail(AOTO_ERR_ARGUMENT, "argmax_finish: the embedding gather needs 16-byte aligned rows, hidden %% 8 == 0");
  if (rope_rows && (!step_state || !cos_table || !sin_table || head_dim <= 0 || head_dim > 256))
    return fail(AOTO_ERR_ARGUMENT, "argmax_finish: RoPE rows need the step state, both tables and "
                "0 < head_dim <= 256");
  // the kernel takes the capacity and head size packed (cap | head_dim << 22)
  if (capacity >= (1 << 22)) return fail(AOTO_ERR_UNSUPPORTED, "argmax_finish: capacity must be below 2^22");
  const int cap_hd = (capacity > 0 ? capacity : 0) | ((rope_rows ? head_dim : 0) << 22);
  return launch("aoto_argmax_finish", dim3(1), dim3(256), 0, stream, keys, step_state, cos_table, sin_table, history,
                history_len, key_count, cap_hd, rope_rows, token_out, embedding, (long long)embedding_rows, hidden,
                hidden_out, error);
}

size_t aoto_hip_w4_gemv_finish_max_keys(void) { return 2048; }

int aoto_hip_w4_gemv_finish(const uint64_t* keys, int key_count, const void* embedding, int64_t embedding_rows,
                            const int32_t* words, const void* scales, const void* norm_weight, float eps,
                            const void* bias, float alpha, float beta, void* y, int K, int N, int group,
                            int64_t* token_out, int64_t* history, int* history_len, int32_t* step_state,
                            int capacity, const void* cos_table, const void* sin_table, int head_dim,
                            void* rope_rows, void* hidden_out, int* error, void* stream) {
  if (!keys || !embedding || !words || !scales || !norm_weight || !y || !token_out || !hidden_out)
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv_finish: null pointer");
  if (key_count <= 0 || (size_t)key_count > aoto_hip_w4_gemv_finish_max_keys())
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv_finish: %d keys, the prologue takes 1 .. %zu", key_count,
                aoto_hip_w4_gemv_finish_max_keys());
  if (embedding_rows <= 0 || N <= 0 || K <= 0)
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv_finish: empty shape K=%d N=%d rows=%lld", K, N, (long long)embedding_rows);
  if ((history == nullptr) != (history_len == nullptr))
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv_finish: a token history needs both pointers");
  if (step_state && (capacity <= 0 || capacity >= (1 << 22)))
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv_finish: step state needs a capacity in (0, 2^22)");
  if (rope_rows && (!step_state || !cos_table || !sin_table || head_dim <= 0 || head_dim > 256))
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv_finish: RoPE rows need the step state, both tables and "
                "0 < head_dim <= 256");
  StreamShape ss{};
  const bool pow2_group = group > 0 && (group & (group - 1)) == 0;
  if (!pow2_group || group < 32 || K % group != 0 || (K / group) % 2 != 0 || !stream_shape(K, N, false, &ss) ||
      !ss.block_x || ss.lpr != 32 || (ss.cpl != 1 && ss.cpl != 4) || ss.rows != 0)
    return fail(AOTO_ERR_UNSUPPORTED, "w4_gemv_finish: the finish prologue is built for the block-staged "
                "q/k/v GEMV shapes (K = 896 or 4096, N <= 16384, power-of-two groups; K=%d N=%d group=%d)",
                K, N, group);
  if (!aligned16(embedding) || !aligned16(words) || !aligned16(norm_weight) || !aligned16(hidden_out) ||
      !aligned4(scales) || !aligned8(keys) || (bias && (N % 2 != 0 || !aligned4(bias))))
    return fail(AOTO_ERR_ARGUMENT, "w4_gemv_finish: embedding, words, norm weight and hidden_out must be 16-byte "
                "aligned, scales and bias 4-byte (N even with a bias), keys 8-byte");
  const StreamLaunch l = stream_launch(ss, K, N, group);
  if (l.shift > 15 || l.wpb > 255) return fail(AOTO_ERR_UNSUPPORTED, "w4_gemv_finish: launch shape out of range");
  aoto::GemvFinishArgs fin{};
  fin.token_out = reinterpret_cast<long long*>(token_out);
  fin.history = reinterpret_cast<long long*>(history);
  fin.history_len = history_len;
  fin.step = step_state;
  fin.cos_table = static_cast<const uint16_t*>(cos_table);
  fin.sin_table = static_cast<const uint16_t*>(sin_table);
  fin.rope_rows = static_cast<uint16_t*>(rope_rows);
  fin.hidden_out = static_cast<uint16_t*>(hidden_out);
  fin.error = error;
  fin.embed_rows = (long long)embedding_rows;
  fin.count = key_count;
  fin.cap = step_state ? capacity : 0;
  fin.head_dim = rope_rows ? head_dim : 0;
  const int shape = l.shift | (l.wpb << 4) | (key_count << 12);
  char name[64];
  snprintf(name, sizeof(name), "aoto_w4_gemv_x%dx%d_n1_b%d_finish", ss.lpr, ss.cpl, bias ? 1 : 0);
  return launch(name, dim3((unsigned)l.grid), dim3(64 * l.wpb), l.shared, stream, keys, words, scales, embedding, K,
                N, shape, bias, norm_weight, eps, alpha, beta, y, fin);
}

int aoto_hip_argmax(const void* logits, int rows, int n, int64_t row_stride, int64_t* out, int64_t* history,
                    int* history_len, void* stream) {
  if (!logits || !out) return fail(AOTO_ERR_ARGUMENT, "argmax: null pointer");
  if (rows <= 0 || n <= 0 || row_stride < n) return fail(AOTO_ERR_ARGUMENT, "argmax: bad shape");
  if ((history == nullptr) != (history_len == nullptr) || (history != nullptr && rows != 1))
    return fail(AOTO_ERR_ARGUMENT, "argmax: a token history needs one row and both pointers");
  return launch("aoto_argmax", dim3(rows), dim3(1024), 0, stream, logits, n, (long long)row_stride, out, history,
                history_len);
}

}  // extern "C"

// ---------------------------------------------------------------- generic graph kernels
namespace {

bool valid_dtype(int dt) { return dt >= AOTO_DT_F32 && dt <= AOTO_DT_I8; }
bool float_dtype(int dt) { return dt == AOTO_DT_F32 || dt == AOTO_DT_BF16; }

long long numel(const aoto_tensor* t) {
  long long n = 1;
  for (int d = 0; d < t->ndim; ++d) n *= t->shape[d];
  return n;
}

int check_tensor(const char* what, const char* name, const aoto_tensor* t, bool allow_scalar) {
  if (t == nullptr) return fail(AOTO_ERR_ARGUMENT, "%s: %s is null", what, name);
  if (t->ndim < 0 || t->ndim > AOTO_MAX_DIMS)
    return fail(AOTO_ERR_ARGUMENT, "%s: %s has %d dims (at most %d)", what, name, t->ndim, AOTO_MAX_DIMS);
  if (t->data == nullptr) {
    if (allow_scalar && t->ndim == 0) return AOTO_OK;
    return fail(AOTO_ERR_ARGUMENT, "%s: %s has no data", what, name);
  }
  if (!valid_dtype(t->dtype)) return fail(AOTO_ERR_ARGUMENT, "%s: %s has element type %d", what, name, t->dtype);
  for (int d = 0; d < t->ndim; ++d)
    if (t->shape[d] < 0) return fail(AOTO_ERR_ARGUMENT, "%s: %s has a negative extent", what, name);
  return AOTO_OK;
}

bool contiguous(const aoto_tensor* t) {
  long long expect = 1;
  for (int d = t->ndim - 1; d >= 0; --d) {
    if (t->shape[d] != 1 && t->strides[d] != expect) return false;
    expect *= t->shape[d];
  }
  return true;
}

// Right-aligned numpy broadcast of `t` onto `out`'s shape: element strides per output dim.
int broadcast_operand(const char* what, const char* name, const aoto_tensor* t, const aoto_tensor* out,
                      aoto::Operand* o) {
  memset(o, 0, sizeof(*o));
  if (t == nullptr) return AOTO_OK;
  if (int s = check_tensor(what, name, t, true)) return s;
  o->data = t->data;
  o->dtype = t->dtype;
  o->value = t->value;
  if (t->data == nullptr) return AOTO_OK;
  if (t->ndim > out->ndim) return fail(AOTO_ERR_ARGUMENT, "%s: %s has more dims than the output", what, name);
  const int shift = out->ndim - t->ndim;
  for (int d = 0; d < t->ndim; ++d) {
    const long long ext = t->shape[d], oext = out->shape[d + shift];
    if (ext == oext)
      o->strides[d + shift] = ext == 1 ? 0 : t->strides[d];
    else if (ext == 1)
      o->strides[d + shift] = 0;
    else
      return fail(AOTO_ERR_ARGUMENT, "%s: %s dim %d (%lld) does not broadcast to %lld", what, name, d, ext, oext);
  }
  return AOTO_OK;
}

unsigned grid_for(long long total) {
  long long blocks = (total + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 8192) blocks = 8192;
  return (unsigned)blocks;
}

}  // namespace

extern "C" {

int aoto_hip_generic_elementwise(int op, const aoto_tensor* out, const aoto_tensor* a, const aoto_tensor* b,
                                 const aoto_tensor* c, double alpha, void* stream) {
  const char* what = "generic_elementwise";
  if (int s = check_tensor(what, "out", out, false)) return s;
  if (!contiguous(out)) return fail(AOTO_ERR_ARGUMENT, "%s: out must be contiguous", what);
  const int arity = op == AOTO_EW_WHERE ? 3 : (op >= AOTO_EW_ADD && op != AOTO_EW_ISNAN ? 2 : 1);
  if (op < 0 || (op > AOTO_EW_BITWISE_NOT && op < AOTO_EW_ADD) || (op > AOTO_EW_LOG_OR && op < AOTO_EW_EQ) ||
      (op > AOTO_EW_ISNAN && op != AOTO_EW_WHERE))
    return fail(AOTO_ERR_ARGUMENT, "%s: unknown op %d", what, op);
  if (a == nullptr || (arity >= 2 && b == nullptr) || (arity == 3 && c == nullptr))
    return fail(AOTO_ERR_ARGUMENT, "%s: op %d takes %d operands", what, op, arity);
  if (op == AOTO_EW_BITWISE_NOT && out->dtype == AOTO_DT_BOOL) op = AOTO_EW_LOGICAL_NOT;  // ~ of bool is not
  aoto::EwArgs args;
  memset(&args, 0, sizeof(args));
  if (int s = broadcast_operand(what, "a", a, out, &args.in[0])) return s;
  if (int s = broadcast_operand(what, "b", arity >= 2 ? b : nullptr, out, &args.in[1])) return s;
  if (int s = broadcast_operand(what, "c", arity == 3 ? c : nullptr, out, &args.in[2])) return s;
  const bool compare = op >= AOTO_EW_EQ && op <= AOTO_EW_ISNAN;
  if (compare) {
    if (out->dtype != AOTO_DT_BOOL) return fail(AOTO_ERR_ARGUMENT, "%s: a comparison writes bool", what);
    args.domain = 2;
  } else if (op == AOTO_EW_WHERE) {
    args.domain = 3;
  } else if (float_dtype(out->dtype)) {
    if (op == AOTO_EW_LOGICAL_NOT || op == AOTO_EW_BITWISE_NOT || (op >= AOTO_EW_BIT_AND && op <= AOTO_EW_LOG_OR))
      return fail(AOTO_ERR_ARGUMENT, "%s: op %d has no floating-point form", what, op);
    args.domain = 0;
  } else {
    const bool int_ok = op == AOTO_EW_CAST || op == AOTO_EW_NEG || op == AOTO_EW_ABS || op == AOTO_EW_LOGICAL_NOT ||
                        op == AOTO_EW_BITWISE_NOT || op == AOTO_EW_ADD || op == AOTO_EW_SUB || op == AOTO_EW_MUL ||
                        op == AOTO_EW_DIV_TRUNC || op == AOTO_EW_DIV_FLOOR || op == AOTO_EW_MAXIMUM ||
                        op == AOTO_EW_MINIMUM || op == AOTO_EW_REMAINDER || (op >= AOTO_EW_BIT_AND && op <= AOTO_EW_LOG_OR);
    if (!int_ok) return fail(AOTO_ERR_ARGUMENT, "%s: op %d has no integer form", what, op);
    // a float operand cast to an integer output truncates: load it as float
    args.domain = (op == AOTO_EW_CAST && a->data && float_dtype(a->dtype)) ? 0 : 1;
  }
  args.op = op;
  args.ndim = out->ndim;
  args.out_dtype = out->dtype;
  args.total = numel(out);
  for (int d = 0; d < out->ndim; ++d) args.shape[d] = out->shape[d];
  args.out = out->data;
  args.alpha = alpha;
  if (args.total == 0) return AOTO_OK;
  return launch("aoto_generic_elementwise", dim3(grid_for(args.total)), dim3(256), 0, stream, args);
}

int aoto_hip_generic_reduce(int op, const aoto_tensor* out, const aoto_tensor* in, void* stream) {
  const char* what = "generic_reduce";
  if (int s = check_tensor(what, "in", in, false)) return s;
  if (int s = check_tensor(what, "out", out, false)) return s;
  if (op < AOTO_RED_SUM || op > AOTO_RED_CUMSUM) return fail(AOTO_ERR_ARGUMENT, "%s: unknown op %d", what, op);
  if (in->ndim < 1) return fail(AOTO_ERR_ARGUMENT, "%s: the input needs a dim to reduce", what);
  const long long len = in->shape[in->ndim - 1];
  const long long total = numel(in);
  const long long rows = len > 0 ? total / len : 0;
  // the leading dims of `in` must collapse to one row stride
  long long row_stride = 0;
  {
    long long expect = -1, extent = 1;
    for (int d = in->ndim - 2; d >= 0; --d) {
      if (in->shape[d] == 1) continue;
      if (expect >= 0 && in->strides[d] != expect)
        return fail(AOTO_ERR_ARGUMENT, "%s: the leading dims of the input do not collapse to one stride", what);
      if (expect < 0) row_stride = in->strides[d];
      expect = in->strides[d] * in->shape[d];
      extent *= in->shape[d];
    }
    (void)extent;
  }
  const bool full = op == AOTO_RED_SOFTMAX || op == AOTO_RED_LOG_SOFTMAX || op == AOTO_RED_CUMSUM;
  if (!contiguous(out) || numel(out) != (full ? total : rows))
    return fail(AOTO_ERR_ARGUMENT, "%s: out must be contiguous with %lld elements", what, full ? total : rows);
  aoto::ReduceArgs args;
  memset(&args, 0, sizeof(args));
  args.op = op;
  const bool int_out = !float_dtype(out->dtype);
  args.domain = (op == AOTO_RED_SUM || op == AOTO_RED_AMAX || op == AOTO_RED_AMIN || op == AOTO_RED_CUMSUM) && int_out
                    ? 1
                    : 0;
  if ((op == AOTO_RED_MEAN || op == AOTO_RED_SOFTMAX || op == AOTO_RED_LOG_SOFTMAX) && int_out)
    return fail(AOTO_ERR_ARGUMENT, "%s: op %d writes a floating-point output", what, op);
  if (op == AOTO_RED_CUMSUM && len > 256 * 4096)
    return fail(AOTO_ERR_UNSUPPORTED, "%s: cumsum rows longer than 1048576", what);
  args.in_dtype = in->dtype;
  args.out_dtype = out->dtype;
  args.rows = rows;
  args.len = len;
  args.in = in->data;
  args.in_row_stride = row_stride;
  args.in_elem_stride = in->strides[in->ndim - 1];
  args.out = out->data;
  args.out_row_stride = full ? len : 1;
  args.out_elem_stride = 1;
  if (rows == 0) return AOTO_OK;
  if (len == 0) {
    if (full) return AOTO_OK;
    return fail(AOTO_ERR_UNSUPPORTED, "%s: reducing an empty dim", what);
  }
  const unsigned grid = (unsigned)(rows < 65536 ? rows : 65536);
  return launch("aoto_generic_reduce", dim3(grid), dim3(256), 0, stream, args);
}

int aoto_hip_generic_matmul(const aoto_tensor* out, const aoto_tensor* a, const aoto_tensor* b,
                            const aoto_tensor* bias, float alpha, float beta, void* stream) {
  const char* what = "generic_matmul";
  if (int s = check_tensor(what, "a", a, false)) return s;
  if (int s = check_tensor(what, "b", b, false)) return s;
  if (int s = check_tensor(what, "out", out, false)) return s;
  if (a->ndim != 3 || b->ndim != 3 || out->ndim != 3)
    return fail(AOTO_ERR_ARGUMENT, "%s: a, b and out must be 3-D [batch, rows, cols]", what);
  const long long B = out->shape[0], M = out->shape[1], N = out->shape[2], K = a->shape[2];
  if ((a->shape[0] != B && a->shape[0] != 1) || (b->shape[0] != B && b->shape[0] != 1) || a->shape[1] != M ||
      b->shape[1] != K || b->shape[2] != N)
    return fail(AOTO_ERR_ARGUMENT, "%s: shapes [%lld,%lld,%lld] x [%lld,%lld,%lld] -> [%lld,%lld,%lld] disagree", what,
                (long long)a->shape[0], (long long)a->shape[1], (long long)a->shape[2], (long long)b->shape[0],
                (long long)b->shape[1], (long long)b->shape[2], B, M, N);
  if (!float_dtype(a->dtype) || !float_dtype(b->dtype) || !float_dtype(out->dtype))
    return fail(AOTO_ERR_UNSUPPORTED, "%s: f32 / bf16 operands only", what);
  if (B > 65535 || (M + 63) / 64 > 65535) return fail(AOTO_ERR_UNSUPPORTED, "%s: grid too large", what);
  aoto::GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.a = a->data;
  g.b = b->data;
  g.c = out->data;
  g.a_dtype = a->dtype;
  g.b_dtype = b->dtype;
  g.c_dtype = out->dtype;
  g.batch = B;
  g.m = M;
  g.n = N;
  g.k = K;
  g.sa_b = a->shape[0] == 1 ? 0 : a->strides[0];
  g.sa_m = a->strides[1];
  g.sa_k = a->strides[2];
  g.sb_b = b->shape[0] == 1 ? 0 : b->strides[0];
  g.sb_k = b->strides[1];
  g.sb_n = b->strides[2];
  g.sc_b = out->strides[0];
  g.sc_m = out->strides[1];
  g.sc_n = out->strides[2];
  g.alpha = alpha;
  g.beta = beta;
  if (bias != nullptr) {
    aoto::Operand o;
    if (int s = broadcast_operand(what, "bias", bias, out, &o)) return s;
    if (o.data == nullptr) return fail(AOTO_ERR_ARGUMENT, "%s: bias needs data", what);
    g.bias = o.data;
    g.bias_dtype = o.dtype;
    g.sbias_b = o.strides[0];
    g.sbias_m = o.strides[1];
    g.sbias_n = o.strides[2];
  }
  if (B == 0 || M == 0 || N == 0) return AOTO_OK;
  return launch("aoto_generic_gemm", dim3((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64), (unsigned)B),
                dim3(256), 0, stream, g);
}

int aoto_hip_generic_index(const aoto_tensor* out, const aoto_tensor* src, int nidx,
                           const aoto_tensor* const* indices, int* error, void* stream) {
  const char* what = "generic_index";
  if (int s = check_tensor(what, "src", src, false)) return s;
  if (int s = check_tensor(what, "out", out, false)) return s;
  if (nidx < 1 || nidx > 4 || nidx > src->ndim || indices == nullptr)
    return fail(AOTO_ERR_ARGUMENT, "%s: 1..4 index tensors over the source's leading dims", what);
  if (!contiguous(src) || !contiguous(out) || src->dtype != out->dtype)
    return fail(AOTO_ERR_ARGUMENT, "%s: src and out must be contiguous and of one element type", what);
  const int rest = src->ndim - nidx;
  const int bdims = out->ndim - rest;
  if (bdims < 0 || bdims > AOTO_MAX_DIMS) return fail(AOTO_ERR_ARGUMENT, "%s: output rank does not fit", what);
  long long inner = 1;
  for (int d = 0; d < rest; ++d) {
    if (out->shape[bdims + d] != src->shape[nidx + d])
      return fail(AOTO_ERR_ARGUMENT, "%s: trailing dims of out and src differ", what);
    inner *= src->shape[nidx + d];
  }
  aoto::IndexArgs args;
  memset(&args, 0, sizeof(args));
  args.src = src->data;
  args.dtype = src->dtype;
  args.nidx = nidx;
  args.bdims = bdims;
  for (int d = 0; d < bdims; ++d) args.bshape[d] = out->shape[d];
  aoto_tensor bshape_view;
  memset(&bshape_view, 0, sizeof(bshape_view));
  bshape_view.ndim = bdims;
  for (int d = 0; d < bdims; ++d) bshape_view.shape[d] = out->shape[d];
  for (int j = 0; j < nidx; ++j) {
    const aoto_tensor* ix = indices[j];
    if (int s = check_tensor(what, "index", ix, false)) return s;
    if (float_dtype(ix->dtype)) return fail(AOTO_ERR_ARGUMENT, "%s: index tensors must be integer or bool", what);
    aoto::Operand o;
    if (int s = broadcast_operand(what, "index", ix, &bshape_view, &o)) return s;
    args.idx[j] = ix->data;
    args.idx_dtype[j] = ix->dtype;
    for (int d = 0; d < bdims; ++d) args.idx_strides[j][d] = o.strides[d];
    args.dim_size[j] = src->shape[j];
    args.src_stride[j] = src->strides[j];
  }
  args.inner = inner;
  args.total = numel(out);
  args.out = out->data;
  args.error = error;
  if (args.total == 0) return AOTO_OK;
  return launch("aoto_generic_index", dim3(grid_for(args.total)), dim3(256), 0, stream, args);
}

int aoto_hip_generic_copy(const aoto_tensor* dst, const aoto_tensor* src, void* stream) {
  const char* what = "generic_copy";
  if (int s = check_tensor(what, "src", src, false)) return s;
  if (int s = check_tensor(what, "dst", dst, false)) return s;
  if (src->ndim != dst->ndim) return fail(AOTO_ERR_ARGUMENT, "%s: src and dst ranks differ", what);
  aoto::CopyArgs args;
  memset(&args, 0, sizeof(args));
  for (int d = 0; d < dst->ndim; ++d) {
    if (src->shape[d] != dst->shape[d]) return fail(AOTO_ERR_ARGUMENT, "%s: src and dst shapes differ", what);
    args.shape[d] = dst->shape[d];
    args.src_strides[d] = src->strides[d];
    args.dst_strides[d] = dst->strides[d];
  }
  args.src = src->data;
  args.dst = dst->data;
  args.src_dtype = src->dtype;
  args.dst_dtype = dst->dtype;
  args.ndim = dst->ndim;
  args.total = numel(dst);
  if (args.total == 0) return AOTO_OK;
  return launch("aoto_generic_copy", dim3(grid_for(args.total)), dim3(256), 0, stream, args);
}

int aoto_hip_generic_fill(const aoto_tensor* dst, double start, double step, void* stream) {
  const char* what = "generic_fill";
  if (int s = check_tensor(what, "dst", dst, false)) return s;
  if (!contiguous(dst)) return fail(AOTO_ERR_ARGUMENT, "%s: dst must be contiguous", what);
  aoto::FillArgs args;
  memset(&args, 0, sizeof(args));
  args.dst = dst->data;
  args.dtype = dst->dtype;
  args.integer = float_dtype(dst->dtype) ? 0 : 1;
  args.total = numel(dst);
  args.start = start;
  args.step = step;
  args.start_i = (long long)start;
  args.step_i = (long long)step;
  if (args.total == 0) return AOTO_OK;
  return launch("aoto_generic_fill", dim3(grid_for(args.total)), dim3(256), 0, stream, args);
}

int aoto_hip_generic_rms_norm(const aoto_tensor* out, const aoto_tensor* x, const aoto_tensor* weight, float eps,
                              int mid_dtype, void* stream) {
  const char* what = "generic_rms_norm";
  if (int s = check_tensor(what, "x", x, false)) return s;
  if (int s = check_tensor(what, "out", out, false)) return s;
  if (x->ndim < 1 || !contiguous(x) || !contiguous(out) || numel(x) != numel(out))
    return fail(AOTO_ERR_ARGUMENT, "%s: x and out must be contiguous and of one size", what);
  if (!float_dtype(x->dtype) || !float_dtype(out->dtype) || !float_dtype(mid_dtype))
    return fail(AOTO_ERR_UNSUPPORTED, "%s: f32 / bf16 only", what);
  const long long hidden = x->shape[x->ndim - 1];
  aoto::RmsArgs args;
  memset(&args, 0, sizeof(args));
  if (weight != nullptr) {
    if (int s = check_tensor(what, "weight", weight, false)) return s;
    if (numel(weight) != hidden || !contiguous(weight) || !float_dtype(weight->dtype))
      return fail(AOTO_ERR_ARGUMENT, "%s: weight must be a contiguous float vector of %lld", what, hidden);
    args.w = weight->data;
    args.w_dtype = weight->dtype;
    args.has_weight = 1;
  }
  args.x = x->data;
  args.out = out->data;
  args.x_dtype = x->dtype;
  args.mid_dtype = mid_dtype;
  args.out_dtype = out->dtype;
  args.hidden = hidden;
  args.rows = hidden > 0 ? numel(x) / hidden : 0;
  args.eps = eps;
  if (args.rows == 0) return AOTO_OK;
  const unsigned grid = (unsigned)(args.rows < 65536 ? args.rows : 65536);
  return launch("aoto_generic_rms_norm", dim3(grid), dim3(256), 0, stream, args);
}

int aoto_hip_generic_attention(const aoto_tensor* out, const aoto_tensor* q, const aoto_tensor* k,
                               const aoto_tensor* v, const aoto_tensor* mask, int causal, float scale,
                               void* stream) {
  const char* what = "generic_attention";
  if (int s = check_tensor(what, "q", q, false)) return s;
  if (int s = check_tensor(what, "k", k, false)) return s;
  if (int s = check_tensor(what, "v", v, false)) return s;
  if (int s = check_tensor(what, "out", out, false)) return s;
  if (q->ndim != 4 || k->ndim != 4 || v->ndim != 4 || out->ndim != 4)
    return fail(AOTO_ERR_ARGUMENT, "%s: q, k, v, out must be 4-D [batch, heads, tokens, dim]", what);
  const long long B = q->shape[0], H = q->shape[1], Lq = q->shape[2], D = q->shape[3];
  const long long Hk = k->shape[1], Lk = k->shape[2], Dv = v->shape[3];
  if (k->shape[0] != B || v->shape[0] != B || v->shape[1] != Hk || v->shape[2] != Lk || k->shape[3] != D ||
      Hk <= 0 || H % Hk != 0)
    return fail(AOTO_ERR_ARGUMENT, "%s: q/k/v shapes disagree", what);
  if (out->shape[0] != B || out->shape[1] != H || out->shape[2] != Lq || out->shape[3] != Dv || !contiguous(out))
    return fail(AOTO_ERR_ARGUMENT, "%s: out must be contiguous [B, H, Lq, Dv]", what);
  if (Lk > 8192) return fail(AOTO_ERR_UNSUPPORTED, "%s: at most 8192 keys (got %lld)", what, Lk);
  if (B * H > 65535 || Lq > 2147483647LL) return fail(AOTO_ERR_UNSUPPORTED, "%s: grid too large", what);
  if (!float_dtype(q->dtype) || !float_dtype(k->dtype) || !float_dtype(v->dtype) || !float_dtype(out->dtype))
    return fail(AOTO_ERR_UNSUPPORTED, "%s: f32 / bf16 only", what);
  aoto::AttnArgs args;
  memset(&args, 0, sizeof(args));
  args.q = q->data;
  args.k = k->data;
  args.v = v->data;
  args.out = out->data;
  args.q_dtype = q->dtype;
  args.k_dtype = k->dtype;
  args.v_dtype = v->dtype;
  args.out_dtype = out->dtype;
  args.causal = causal;
  args.batch = (int)B;
  args.heads = (int)H;
  args.kv_heads = (int)Hk;
  args.lq = (int)Lq;
  args.lk = (int)Lk;
  args.d = (int)D;
  args.dv = (int)Dv;
  for (int d = 0; d < 4; ++d) {
    args.qs[d] = q->strides[d];
    args.ks[d] = k->strides[d];
    args.vs[d] = v->strides[d];
  }
  if (mask != nullptr) {
    aoto_tensor shape4;
    memset(&shape4, 0, sizeof(shape4));
    shape4.ndim = 4;
    shape4.shape[0] = B;
    shape4.shape[1] = H;
    shape4.shape[2] = Lq;
    shape4.shape[3] = Lk;
    aoto::Operand o;
    if (int s = broadcast_operand(what, "mask", mask, &shape4, &o)) return s;
    if (o.data == nullptr) return fail(AOTO_ERR_ARGUMENT, "%s: mask needs data", what);
    if (o.dtype != AOTO_DT_BOOL && !float_dtype(o.dtype))
      return fail(AOTO_ERR_ARGUMENT, "%s: mask must be bool or float", what);
    args.mask = o.data;
    args.mask_dtype = o.dtype;
    for (int d = 0; d < 4; ++d) args.ms[d] = o.strides[d];
  }
  args.scale = scale;
  if (B == 0 || H == 0 || Lq == 0) return AOTO_OK;
  return launch("aoto_generic_attention", dim3((unsigned)Lq, (unsigned)(B * H)), dim3(256), 0, stream, args);
}

}  // extern "C"
