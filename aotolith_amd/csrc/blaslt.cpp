// Plain bf16 GEMMs on hipBLASLt for long prefills (host code of libaoto_hip.so).
//
//   D[M][N] = X[M][K] . W[N][K]^T (+ bias[N]) (+ C[M][N]),  f32 accumulation,
//   D bf16 (one rounding of the f32 sum) or f32.
//
// The prefill of a long prompt takes this path after unpacking its packed
// weight to bf16 (the reference's own prefill form: unpack per call, then a
// plain GEMM, models/quantized.py:61-76): at 1024+ rows the hand-written
// fused-dequant GEMM is bound by its dequant VALU (one exact bf16(code*scale)
// per weight; MFMA ~33% busy) while the unpacked weight feeds hipBLASLt's MFMA
// kernels at 1.1-1.3 PFLOP/s on random data (52-60% MFMA busy, Llama-3-8B
// projections at 2048 rows).
//
// hipBLASLt is column-major: D^T (N x M, ld N) = op(A) . B with A = W read as
// the K x N column-major matrix (ld K) and transposed, B = X read as the K x M
// column-major matrix (ld K) - the row-major tensors as they lie in memory.
// Algorithms are asked for with no workspace: a workspace-using algorithm may
// clear it with a memset node when a caller captures the launch in a graph.
// The heuristic's first pick is often not the fastest on this device (Llama-3-8B
// at 2048 rows, random data: o 72.5 -> 55.4 us, down 228.6 -> 181.8 us for the
// best of its first 12 workspace-free candidates), so the first call of a shape
// outside a graph capture times up to kCandidates of them on the call's own x
// and w, into a scratch output the caller provides (a region of its workspace
// that the call overwrites anyway), and keeps the fastest.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "aoto_hip.h"
#include "internal.h"

namespace aoto {
namespace {

struct LtKey {
  int device, M, N, K, d_f32, bias, c;
  bool operator<(const LtKey& o) const {
    return std::tie(device, M, N, K, d_f32, bias, c) < std::tie(o.device, o.M, o.N, o.K, o.d_f32, o.bias, o.c);
  }
};

constexpr int kCandidates = 12;

struct LtPlan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr, d = nullptr;
  std::vector<hipblasLtMatmulAlgo_t> candidates;  // workspace-free, heuristic order
  hipblasLtMatmulAlgo_t algo{};
  bool tuned = false;
};

std::mutex g_lt_mutex;
std::map<int, hipblasLtHandle_t> g_lt_handles;
std::map<LtKey, LtPlan> g_lt_plans;

int lt_fail(hipblasStatus_t st, const char* what) {
  return set_error(AOTO_ERR_HIP, "hipBLASLt %s failed (status %d)", what, (int)st);
}

// With g_lt_mutex held.
int lt_handle(int device, hipblasLtHandle_t* handle) {
  auto it = g_lt_handles.find(device);
  if (it == g_lt_handles.end()) {
    hipblasLtHandle_t h = nullptr;
    if (hipblasStatus_t st = hipblasLtCreate(&h)) return lt_fail(st, "handle creation");
    it = g_lt_handles.emplace(device, h).first;
  }
  *handle = it->second;
  return AOTO_OK;
}

// With g_lt_mutex held: the cached descriptor, layouts and algorithm of a shape.
int lt_plan(hipblasLtHandle_t handle, const LtKey& key, LtPlan** plan) {
  auto it = g_lt_plans.find(key);
  if (it != g_lt_plans.end()) {
    *plan = &it->second;
    return AOTO_OK;
  }
  LtPlan p;
  if (hipblasStatus_t st = hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F))
    return lt_fail(st, "descriptor creation");
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
  hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
  if (key.bias) {
    const hipblasLtEpilogue_t epilogue = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bias_type = HIP_R_16BF;
    hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epilogue, sizeof(epilogue));
    hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bias_type, sizeof(bias_type));
  }
  const hipDataType dtype = key.d_f32 ? HIP_R_32F : HIP_R_16BF;
  hipblasStatus_t st = hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, key.K, key.N, key.K);
  if (!st) st = hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, key.K, key.M, key.K);
  // C is the residual (bf16) when given, else D itself with beta = 0
  if (!st) st = hipblasLtMatrixLayoutCreate(&p.c, key.c ? HIP_R_16BF : dtype, key.N, key.M, key.N);
  if (!st) st = hipblasLtMatrixLayoutCreate(&p.d, dtype, key.N, key.M, key.N);
  if (st) return lt_fail(st, "layout creation");
  hipblasLtMatmulPreference_t pref = nullptr;
  if ((st = hipblasLtMatmulPreferenceCreate(&pref))) return lt_fail(st, "preference creation");
  const uint64_t no_workspace = 0;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &no_workspace,
                                        sizeof(no_workspace));
  hipblasLtMatmulHeuristicResult_t results[kCandidates] = {};
  int found = 0;
  st = hipblasLtMatmulAlgoGetHeuristic(handle, p.op, p.a, p.b, p.c, p.d, pref, kCandidates, results, &found);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (st) return lt_fail(st, "algorithm search");
  for (int i = 0; i < found; ++i)
    if (results[i].workspaceSize == 0) p.candidates.push_back(results[i].algo);
  if (p.candidates.empty())
    return set_error(AOTO_ERR_UNSUPPORTED, "hipBLASLt has no workspace-free algorithm for M=%d N=%d K=%d", key.M,
                     key.N, key.K);
  p.algo = p.candidates[0];
  *plan = &g_lt_plans.emplace(key, p).first->second;
  return AOTO_OK;
}

// With g_lt_mutex held: time each candidate (one warm-up, then 3 launches between
// events) on the call's x, w and bias into the zeroed scratch output (M * N of the
// output type, also the C input when the plan has one) and keep the fastest.
// Nothing is allocated. Not inside a graph capture (nothing may synchronize
// there): the plan stays untuned and the first uncaptured call tunes it. Any
// failure keeps the heuristic's first pick.
void lt_tune(hipblasLtHandle_t handle, const LtKey& key, LtPlan* plan, const void* x, const void* w,
             const void* bias, void* scratch, hipStream_t stream) {
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone) return;
  plan->tuned = true;
  if (plan->candidates.size() < 2 || scratch == nullptr) return;
  const size_t bytes = (size_t)key.M * key.N * (key.d_f32 ? 4 : 2);
  hipEvent_t start = nullptr, stop = nullptr;
  if (hipEventCreate(&start) != hipSuccess || hipEventCreate(&stop) != hipSuccess ||
      hipMemsetAsync(scratch, 0, bytes, stream) != hipSuccess) {
    (void)hipGetLastError();
  } else {
    if (bias != nullptr)
      hipblasLtMatmulDescSetAttribute(plan->op, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
    const float alpha = 1.0f, beta = key.c ? 1.0f : 0.0f;
    float best = 0.f;
    for (const hipblasLtMatmulAlgo_t& algo : plan->candidates) {
      bool ok = true;
      for (int i = 0; i < 4 && ok; ++i) {
        if (i == 1) ok = hipEventRecord(start, stream) == hipSuccess;
        ok = ok && hipblasLtMatmul(handle, plan->op, &alpha, w, plan->a, x, plan->b, &beta, scratch, plan->c,
                                   scratch, plan->d, &algo, nullptr, 0, stream) == HIPBLAS_STATUS_SUCCESS;
      }
      float ms = 0.f;
      ok = ok && hipEventRecord(stop, stream) == hipSuccess && hipEventSynchronize(stop) == hipSuccess &&
           hipEventElapsedTime(&ms, start, stop) == hipSuccess;
      if (ok && (best == 0.f || ms < best)) {
        best = ms;
        plan->algo = algo;
      }
    }
    (void)hipStreamSynchronize(stream);
  }
  if (start != nullptr) (void)hipEventDestroy(start);
  if (stop != nullptr) (void)hipEventDestroy(stop);
}

}  // namespace

int library_prepare(int device) {
  std::lock_guard<std::mutex> lock(g_lt_mutex);
  hipblasLtHandle_t handle = nullptr;
  return lt_handle(device, &handle);
}

int library_gemm(int M, int N, int K, const void* x, const void* w, const void* bias, const void* c, void* d,
                 bool d_f32, void* scratch, void* stream) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return set_error(AOTO_ERR_HIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(g_lt_mutex);
  hipblasLtHandle_t handle = nullptr;
  if (int s = lt_handle(device, &handle)) return s;
  LtPlan* plan = nullptr;
  const LtKey key{device, M, N, K, d_f32 ? 1 : 0, bias != nullptr, c != nullptr};
  if (int s = lt_plan(handle, key, &plan)) return s;
  if (!plan->tuned) lt_tune(handle, key, plan, x, w, bias, scratch, (hipStream_t)stream);
  if (bias != nullptr)
    hipblasLtMatmulDescSetAttribute(plan->op, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
  const float alpha = 1.0f, beta = c != nullptr ? 1.0f : 0.0f;
  const void* cin = c != nullptr ? c : d;
  if (hipblasStatus_t st = hipblasLtMatmul(handle, plan->op, &alpha, w, plan->a, x, plan->b, &beta, cin, plan->c,
                                           d, plan->d, &plan->algo, nullptr, 0, (hipStream_t)stream))
    return lt_fail(st, "matmul");
  return AOTO_OK;
}

}  // namespace aoto
