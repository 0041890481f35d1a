// The engine's projections: y[T, out] = x[T, in] * W^T with W stored [out, in] row-major (a
// PyTorch Linear without bias), fp16 in and out, fp32 accumulation. ref: kernels/linear.cuh:5-7,
// kernels/linear.cu:5-25 (cublasGemmEx, CUBLAS_COMPUTE_32F).
//
// These are plain library GEMMs, so they go to hipBLASLt, except with at most 8 rows (a decode
// step with few sequences), where llmk_linear_rows (gemv.hip) streams the weights itself.
// Viewed column-major, the row-major buffers are W: [in x out] (ld in), x: [in x T] (ld in),
// y: [out x T] (ld out), and y = op_T(W) * x -- the same formulation as the reference's cuBLAS
// call.
//
// A handle owns one hipBLASLt handle, a 32 MiB workspace allocated once at creation, and a
// cache of per-shape plans (descriptors, layouts and the chosen algorithm). The first call of a
// shape takes the heuristic's first algorithm; later calls, including calls made while a stream
// is being captured into a HIP graph, only enqueue the GEMM.
//
// llmk_blas_tune replaces a shape's plan with the fastest of up to kCandidates heuristic
// algorithms, each timed on the caller's stream with the caller's operands (y is overwritten):
// every candidate by its best of kTimedRuns launches, then the kFinalists fastest again by the
// median of kFinalRuns launches (a single cold launch of a 10-30 us GEMM varies by several
// percent, enough to swap plans that differ by 10% inside a decode step).
// Each timed run follows a 512 MiB write that evicts the 256 MB Infinity Cache, because in a
// decode step every weight matrix arrives cold from HBM (2.5 GB of weights stream through per
// step); with warm caches the ranking favours small tiles that lose on cold data. Tuning costs
// tens of milliseconds per shape, so it is for the shapes a caller repeats (its decode batch
// sizes), not for every prompt length.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "llmk.h"

namespace {

constexpr size_t kWorkspaceBytes = 32u << 20;
constexpr int kCandidates = 128;  // heuristic results considered per shape
constexpr int kTimedRuns = 3;     // timed cold launches per candidate (after one untimed)
constexpr int kFinalists = 4;     // candidates timed again
constexpr int kFinalRuns = 15;    // timed cold launches per finalist (median taken)
constexpr size_t kFlushBytes = 512u << 20;

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo;
  size_t ws = 0;
};

void destroy_plan(Plan& p) {
  if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
  if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
  if (p.d) hipblasLtMatrixLayoutDestroy(p.d);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  p = Plan();
}

}  // namespace

struct llmk_blas {
  hipblasLtHandle_t lt = nullptr;
  void* workspace = nullptr;
  int device = 0;
  std::mutex mu;
  std::map<std::tuple<int, int, int>, Plan> plans;
  std::vector<Plan> retired;  // plans replaced by llmk_blas_tune
};

namespace {

// Smallest (median: false) or median (true) duration of `runs` cold launches of one algorithm
// (each after a write of the flush buffer, when there is one), or a negative value if it fails
// to run.
float time_algo(llmk_blas* h, const Plan& q, const hipblasLtMatmulAlgo_t& algo, size_t ws,
                const void* x, const void* w, void* y, void* flush, hipStream_t stream, int runs,
                bool median) {
  const float alpha = 1.0f, beta = 0.0f;
  auto run = [&] {
    return hipblasLtMatmul(h->lt, q.desc, &alpha, w, q.a, x, q.b, &beta, y, q.d, y, q.d, &algo,
                           h->workspace, ws, stream) == HIPBLAS_STATUS_SUCCESS;
  };
  if (!run()) return -1.0f;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0f;
  std::vector<float> t;
  bool ok = true;
  for (int i = 0; ok && i < runs; ++i) {
    if (flush) ok = hipMemsetAsync(flush, i & 0xFF, kFlushBytes, stream) == hipSuccess;
    ok = ok && hipEventRecord(e0, stream) == hipSuccess && run() &&
         hipEventRecord(e1, stream) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
    float ms = 0.0f;
    ok = ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
    if (ok) t.push_back(ms);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (!ok || t.empty()) return -1.0f;
  std::sort(t.begin(), t.end());
  return median ? t[t.size() / 2] : t[0];
}

// Builds the plan of one (T, in, out) shape: the heuristic's first algorithm, or with `tune`
// the fastest candidate timed on `stream` with the call's operands (not while the stream is
// capturing). Returns LLMK_OK or LLMK_ERR_BLAS.
int make_plan(llmk_blas* h, int T, int in, int out, const void* x, const void* w, void* y,
              hipStream_t stream, bool tune, Plan* p) {
  Plan q;
  const hipblasOperation_t opA = HIPBLAS_OP_T, opB = HIPBLAS_OP_N;
  bool ok = hipblasLtMatmulDescCreate(&q.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) ==
                HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatmulDescSetAttribute(q.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opA,
                                            sizeof(opA)) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatmulDescSetAttribute(q.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opB,
                                            sizeof(opB)) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatrixLayoutCreate(&q.a, HIP_R_16F, in, out, in) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatrixLayoutCreate(&q.b, HIP_R_16F, in, T, in) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatrixLayoutCreate(&q.d, HIP_R_16F, out, T, out) == HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (ok) {
    const uint64_t ws = kWorkspaceBytes;
    ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                               &ws, sizeof(ws)) == HIPBLAS_STATUS_SUCCESS;
  }
  if (ok) {
    hipblasLtMatmulHeuristicResult_t res[kCandidates];
    int found = 0;
    ok = hipblasLtMatmulAlgoGetHeuristic(h->lt, q.desc, q.a, q.b, q.d, q.d, pref, kCandidates,
                                         res, &found) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && found > 0;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const bool timed = tune && ok && found > 1 &&
                       hipStreamIsCapturing(stream, &cap) == hipSuccess &&
                       cap == hipStreamCaptureStatusNone;
    int pick = -1;
    void* flush = nullptr;
    if (timed && hipMalloc(&flush, kFlushBytes) != hipSuccess) flush = nullptr;
    std::vector<std::pair<float, int>> first;  // (best of kTimedRuns, candidate)
    for (int i = 0; ok && i < found; ++i) {
      if (res[i].state != HIPBLAS_STATUS_SUCCESS || res[i].workspaceSize > kWorkspaceBytes)
        continue;
      if (!timed) {
        pick = i;
        break;
      }
      const float t = time_algo(h, q, res[i].algo, res[i].workspaceSize, x, w, y, flush, stream,
                                kTimedRuns, false);
      if (t > 0.0f) first.emplace_back(t, i);
    }
    if (timed && !first.empty()) {
      std::sort(first.begin(), first.end());
      float best = 0.0f;
      for (size_t f = 0; f < first.size() && f < (size_t)kFinalists; ++f) {
        const int i = first[f].second;
        const float t = time_algo(h, q, res[i].algo, res[i].workspaceSize, x, w, y, flush,
                                  stream, kFinalRuns, true);
        if (t > 0.0f && (pick < 0 || t < best)) {
          pick = i;
          best = t;
        }
      }
    }
    if (flush) (void)hipFree(flush);
    ok = ok && pick >= 0;
    if (ok) {
      q.algo = res[pick].algo;
      q.ws = res[pick].workspaceSize;
    }
  }
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (!ok) {
    destroy_plan(q);
    return LLMK_ERR_BLAS;
  }
  *p = q;
  return LLMK_OK;
}

}  // namespace

extern "C" int llmk_blas_create(llmk_blas** out) {
  if (!out) return LLMK_ERR_INVALID_VALUE;
  *out = nullptr;
  llmk_blas* h = new llmk_blas();
  int st = (int)hipGetDevice(&h->device);
  if (st == LLMK_OK && hipblasLtCreate(&h->lt) != HIPBLAS_STATUS_SUCCESS) st = LLMK_ERR_BLAS;
  if (st == LLMK_OK) st = (int)hipMalloc(&h->workspace, kWorkspaceBytes);
  if (st != LLMK_OK) {
    if (h->lt) hipblasLtDestroy(h->lt);
    delete h;
    return st;
  }
  *out = h;
  return LLMK_OK;
}

extern "C" void llmk_blas_destroy(llmk_blas* h) {
  if (!h) return;
  for (auto& kv : h->plans) destroy_plan(kv.second);
  for (auto& p : h->retired) destroy_plan(p);
  if (h->workspace) (void)hipFree(h->workspace);
  if (h->lt) hipblasLtDestroy(h->lt);
  delete h;
}

// Whether llmk_linear runs its own few-rows kernel (llmk_linear_rows) for this call.
static bool rows_kernel_applies(const uint16_t* x, const uint16_t* w, int T, int in_features) {
  return T <= LLMK_LINEAR_ROWS_MAX && in_features % 512 == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0;
}

extern "C" int llmk_linear(llmk_blas* h, const uint16_t* x, const uint16_t* w, uint16_t* y, int T,
                           int in_features, int out_features, void* stream) {
  if (!h || T < 0 || in_features <= 0 || out_features <= 0) return LLMK_ERR_INVALID_VALUE;
  if (T == 0) return LLMK_OK;
  if (!x || !w || !y) return LLMK_ERR_INVALID_VALUE;
  if (rows_kernel_applies(x, w, T, in_features))
    return llmk_linear_rows(x, w, y, T, in_features, out_features, stream);
  Plan p;
  {
    std::lock_guard<std::mutex> lock(h->mu);
    auto key = std::make_tuple(T, in_features, out_features);
    auto it = h->plans.find(key);
    if (it == h->plans.end()) {
      const int st = make_plan(h, T, in_features, out_features, x, w, y,
                               static_cast<hipStream_t>(stream), false, &p);
      if (st != LLMK_OK) return st;
      h->plans.emplace(key, p);
    } else {
      p = it->second;
    }
  }
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t st =
      hipblasLtMatmul(h->lt, p.desc, &alpha, w, p.a, x, p.b, &beta, y, p.d, y, p.d, &p.algo,
                      h->workspace, p.ws, static_cast<hipStream_t>(stream));
  return st == HIPBLAS_STATUS_SUCCESS ? LLMK_OK : LLMK_ERR_BLAS;
}

extern "C" int llmk_blas_tune(llmk_blas* h, const uint16_t* x, const uint16_t* w, uint16_t* y,
                              int T, int in_features, int out_features, void* stream) {
  if (!h || T <= 0 || in_features <= 0 || out_features <= 0 || !x || !w || !y)
    return LLMK_ERR_INVALID_VALUE;
  if (rows_kernel_applies(x, w, T, in_features)) return LLMK_OK;  // no library plan to choose
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cap) != hipSuccess ||
      cap != hipStreamCaptureStatusNone)
    return LLMK_ERR_INVALID_VALUE;
  std::lock_guard<std::mutex> lock(h->mu);
  Plan p;
  const int st = make_plan(h, T, in_features, out_features, x, w, y,
                           static_cast<hipStream_t>(stream), true, &p);
  if (st != LLMK_OK) return st;
  auto key = std::make_tuple(T, in_features, out_features);
  auto it = h->plans.find(key);
  if (it != h->plans.end()) {
    // A graph captured earlier may hold the old plan's algorithm by value; its descriptors are
    // kept alive until the handle is destroyed.
    h->retired.push_back(it->second);
    it->second = p;
  } else {
    h->plans.emplace(key, p);
  }
  return LLMK_OK;
}