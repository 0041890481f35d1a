// The engine's projections: y[T, out] = x[T, in] * W^T with W stored [out, in] row-major (a
// PyTorch Linear without bias), fp16 in and out, fp32 accumulation. ref: kernels/linear.cuh:5-7,
// kernels/linear.cu:5-25 (cublasGemmEx, CUBLAS_COMPUTE_32F).
//
// These are plain library GEMMs, so they go to hipBLASLt. Viewed column-major, the row-major
// buffers are W: [in x out] (ld in), x: [in x T] (ld in), y: [out x T] (ld out), and
// y = op_T(W) * x -- the same formulation as the reference's cuBLAS call.
//
// A handle owns one hipBLASLt handle, a 32 MiB workspace allocated once at creation, and a
// cache of per-shape plans (descriptors, layouts, and the heuristic's first algorithm). The
// heuristic query runs on the first call of a shape only; later calls, including calls made
// while a stream is being captured into a HIP graph, only enqueue the GEMM.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "llmk.h"

namespace {

constexpr size_t kWorkspaceBytes = 32u << 20;

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
};

namespace {

// Builds the plan of one (T, in, out) shape. Returns LLMK_OK or LLMK_ERR_BLAS.
int make_plan(llmk_blas* h, int T, int in, int out, Plan* p) {
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
    hipblasLtMatmulHeuristicResult_t res[8];
    int found = 0;
    ok = hipblasLtMatmulAlgoGetHeuristic(h->lt, q.desc, q.a, q.b, q.d, q.d, pref, 8, res,
                                         &found) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && found > 0;
    int pick = -1;
    for (int i = 0; ok && i < found && pick < 0; ++i)
      if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= kWorkspaceBytes)
        pick = i;
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
  if (h->workspace) (void)hipFree(h->workspace);
  if (h->lt) hipblasLtDestroy(h->lt);
  delete h;
}

extern "C" int llmk_linear(llmk_blas* h, const uint16_t* x, const uint16_t* w, uint16_t* y, int T,
                           int in_features, int out_features, void* stream) {
  if (!h || T < 0 || in_features <= 0 || out_features <= 0) return LLMK_ERR_INVALID_VALUE;
  if (T == 0) return LLMK_OK;
  if (!x || !w || !y) return LLMK_ERR_INVALID_VALUE;
  Plan p;
  {
    std::lock_guard<std::mutex> lock(h->mu);
    auto key = std::make_tuple(T, in_features, out_features);
    auto it = h->plans.find(key);
    if (it == h->plans.end()) {
      const int st = make_plan(h, T, in_features, out_features, &p);
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
