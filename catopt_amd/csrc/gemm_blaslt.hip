// Plain bf16 GEMMs through hipBLASLt.
//
// The fused GEMMs of the delivered forms (paired SiLU / GLU epilogues, bias
// spines) run on this library's own MFMA kernels (gemm_bf16.hip).  A GEMM
// with no epilogue is a plain library GEMM, and hipBLASLt's tuned gfx950
// kernels run it faster than ours (C2's down projection, 16384 x 4096 x
// 11008: 0.92 ms against 1.35 ms).  catopt_hip_linear hands such calls here.
//
//   row-major  C[M,N] = A[M,K] · B[N,K]ᵀ
//   = column-major  Cᶜ (N x M) = (Bᶜ)ᵀ · Aᶜ  with Bᶜ = B as K x N (ld ldb),
//     Aᶜ = A as K x M (ld lda), Cᶜ ld ldc:  opA = T on B, opB = N on A.
//
// One handle per device; per shape, the matmul descriptor, layouts and the
// first heuristic algorithm that needs no workspace are cached (nothing
// here allocates device memory per call, and a call records into a hipGraph
// once its shape has been seen).  Any hipBLASLt failure returns false and
// the caller runs its own kernel instead.  CATOPT_HIP_NO_BLASLT=1 disables
// this path (to compare against the in-house kernel).
#include <hipblaslt/hipblaslt.h>

#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>

#include "common.hpp"

namespace catopt {
namespace {

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;
};

using Key = std::tuple<int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t>;

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<Key, Plan> g_plans;

bool disabled() {
  static const bool off = [] {
    const char* e = std::getenv("CATOPT_HIP_NO_BLASLT");
    return e && e[0] && e[0] != '0';
  }();
  return off;
}

// Builds (once) the plan for this device and shape; ok=false when hipBLASLt
// has no algorithm for it.  Called with g_mu held.
Plan* plan_for(int dev, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc) {
  const Key key{dev, M, N, K, lda, ldb, ldc};
  auto it = g_plans.find(key);
  if (it != g_plans.end()) return &it->second;
  Plan& p = g_plans[key];
  hipblasLtHandle_t h = nullptr;
  auto hit = g_handles.find(dev);
  if (hit == g_handles.end()) {
    if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return &p;
    g_handles[dev] = h;
  } else {
    h = hit->second;
  }
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return &p;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  if (hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) != HIPBLAS_STATUS_SUCCESS)
    return &p;
  if (hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, K, N, ldb) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, K, M, lda) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_16BF, N, M, ldc) != HIPBLAS_STATUS_SUCCESS)
    return &p;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return &p;
  const uint64_t no_ws = 0;
  hipblasLtMatmulHeuristicResult_t res[4];
  int n = 0;
  const bool got =
      hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &no_ws,
                                            sizeof(no_ws)) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.la, p.lb, p.lc, p.lc, pref, 4, res, &n) ==
          HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulPreferenceDestroy(pref);
  for (int i = 0; got && i < n; ++i) {
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize == 0) {
      p.algo = res[i].algo;
      p.ok = true;
      break;
    }
  }
  return &p;
}

}  // namespace

bool blaslt_linear_bf16(int64_t M, int64_t N, int64_t K, const void* x, int64_t ldx, const void* w,
                        int64_t ldw, void* y, int64_t ldy, hipStream_t s) {
  if (disabled()) return false;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  hipblasLtHandle_t h = nullptr;
  Plan* p = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    p = plan_for(dev, M, N, K, ldx, ldw, ldy);
    if (!p->ok) return false;
    h = g_handles[dev];
  }
  const float alpha = 1.f, beta = 0.f;
  return hipblasLtMatmul(h, p->desc, &alpha, w, p->la, x, p->lb, &beta, y, p->lc, y, p->lc, &p->algo,
                         nullptr, 0, s) == HIPBLAS_STATUS_SUCCESS;
}

}  // namespace catopt
