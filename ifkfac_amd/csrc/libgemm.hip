// Plain products through hipBLASLt, the vendor GEMM library:
//   C (fp32, row-major M x N, ldc) = alpha * op(A) op(B) + beta * C,
// bf16 operands with K contiguous (A M x K, B N x K) in bf16 arithmetic, and
// fp32 operands stored either way (gemm.h's kc flags) in fp32 arithmetic.
// The engine's dispatcher (gemm.hip) sends here the products that are plain
// in this sense -- no triangular operand, no bf16 copy of the result -- which
// are the Gram columns of a factor update and its panel and band updates:
// for those narrow, long-K shapes (an 11008 x 1024 output at K = 16384) the
// library's tuned kernels run at over twice the rate of the direct-to-LDS
// kernel.  Products with a triangular operand keep the engine's kernels,
// which skip the zero half.
//
// Row-major C = A B^T is the column-major product C^T = B^T-op(B_cm) A_cm:
// the library's "A" is our B viewed column-major (K x N, ld ldb) used
// transposed, its "B" is our A (K x M, ld lda) used as is, and C^T is N x M
// with ld ldc.  One handle per (device, stream), so that products enqueued on
// different streams never share a handle's state, and one plan per (handle,
// shape, strides, beta != 0, workspace): the descriptors and the heuristic's
// first algorithm, made once under a lock and kept for the process (each a
// few hundred bytes of host memory).  Every call gets the caller's split-K
// scratch of the same stream as its workspace, whatever the algorithm asks.
#include <hipblaslt/hipblaslt.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "common.h"
#include "gemm.h"

namespace ifk {

namespace {

struct LtKey {
  int dev;
  uintptr_t stream;
  int64_t m, n, k, lda, ldb, ldc;
  int beta_nz;
  size_t ws;
  int adt, akc, bdt, bkc;   // operand types (DT_F32 / DT_BF16) and K-contiguity
  bool operator<(const LtKey& o) const {
    return std::tie(dev, stream, m, n, k, lda, ldb, ldc, beta_nz, ws, adt, akc, bdt, bkc) <
           std::tie(o.dev, o.stream, o.m, o.n, o.k, o.lda, o.ldb, o.ldc, o.beta_nz, o.ws, o.adt,
                    o.akc, o.bdt, o.bkc);
  }
};

struct LtPlan {
  bool ok = false;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo;
  size_t ws = 0;
};

std::mutex g_lt_mu;
std::map<std::pair<int, uintptr_t>, hipblasLtHandle_t> g_lt_handle;
std::map<LtKey, LtPlan> g_lt_plan;

// the plan for a key (made on first use); null handle when the library
// cannot be initialised on this device
const LtPlan* lt_plan(const LtKey& key, hipblasLtHandle_t* h) {
  std::lock_guard<std::mutex> lock(g_lt_mu);
  const auto hk = std::make_pair(key.dev, key.stream);
  auto hi = g_lt_handle.find(hk);
  if (hi == g_lt_handle.end()) {
    hipblasLtHandle_t nh = nullptr;
    if (hipblasLtCreate(&nh) != HIPBLAS_STATUS_SUCCESS) nh = nullptr;
    hi = g_lt_handle.emplace(hk, nh).first;
  }
  *h = hi->second;
  if (!*h) return nullptr;
  auto it = g_lt_plan.find(key);
  if (it != g_lt_plan.end()) return &it->second;
  LtPlan pl;
  bool ok = hipblasLtMatmulDescCreate(&pl.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) ==
            HIPBLAS_STATUS_SUCCESS;
  // the library's A is our B: K-contiguous B (N x K row-major) is a K x N
  // column-major matrix used transposed, else (K x N row-major) an N x K one
  // used as is; its B is our A: K-contiguous A (M x K row-major) is K x M
  // column-major used as is, else (K x M row-major) M x K used transposed
  const int32_t opA = key.bkc ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  const int32_t opB = key.akc ? HIPBLAS_OP_N : HIPBLAS_OP_T;
  const hipDataType ta = key.bdt == DT_BF16 ? HIP_R_16BF : HIP_R_32F;
  const hipDataType tb = key.adt == DT_BF16 ? HIP_R_16BF : HIP_R_32F;
  ok = ok && hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opA,
                                             sizeof(opA)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opB,
                                             sizeof(opB)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&pl.la, ta, (uint64_t)(key.bkc ? key.k : key.n),
                                         (uint64_t)(key.bkc ? key.n : key.k),
                                         key.ldb) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&pl.lb, tb, (uint64_t)(key.akc ? key.k : key.m),
                                         (uint64_t)(key.akc ? key.m : key.k),
                                         key.lda) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&pl.lc, HIP_R_32F, (uint64_t)key.n, (uint64_t)key.m,
                                         key.ldc) == HIPBLAS_STATUS_SUCCESS;
  if (ok) {
    hipblasLtMatmulPreference_t pref = nullptr;
    ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
    const uint64_t wsb = key.ws;
    ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                     &wsb, sizeof(wsb)) == HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulHeuristicResult_t res[1];
    int count = 0;
    ok = ok && hipblasLtMatmulAlgoGetHeuristic(*h, pl.desc, pl.la, pl.lb, pl.lc, pl.lc, pref, 1,
                                               res, &count) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && count >= 1 && res[0].state == HIPBLAS_STATUS_SUCCESS && res[0].workspaceSize <= key.ws;
    if (ok) {
      pl.algo = res[0].algo;
      pl.ws = res[0].workspaceSize;
    }
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  }
  pl.ok = ok;
  return &g_lt_plan.emplace(key, pl).first->second;
}

}  // namespace

// -1: not yet read from the environment; then 0 / 1
static std::atomic<int> g_lib_on{-1};

bool lib_gemm_enabled() {
  int v = g_lib_on.load(std::memory_order_relaxed);
  if (v < 0) {
    const char* e = std::getenv("IFK_GEMM_LIB");
    int want = (e && std::strcmp(e, "0") == 0) ? 0 : 1;
    g_lib_on.compare_exchange_strong(v, want);
    v = g_lib_on.load(std::memory_order_relaxed);
  }
  return v != 0;
}

int lib_gemm_set(int on) {
  const int prev = lib_gemm_enabled() ? 1 : 0;
  g_lib_on.store(on ? 1 : 0, std::memory_order_relaxed);
  return prev;
}

int lib_gemm_release(hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("release_stream_state: hipGetDevice failed");
    return IFK_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_lt_mu);
  bool ok = true;
  for (auto it = g_lt_plan.begin(); it != g_lt_plan.end();) {
    if (it->first.dev == dev && it->first.stream == (uintptr_t)s) {
      LtPlan& pl = it->second;
      for (hipblasLtMatrixLayout_t l : {pl.la, pl.lb, pl.lc})
        if (l) ok = hipblasLtMatrixLayoutDestroy(l) == HIPBLAS_STATUS_SUCCESS && ok;
      if (pl.desc) ok = hipblasLtMatmulDescDestroy(pl.desc) == HIPBLAS_STATUS_SUCCESS && ok;
      it = g_lt_plan.erase(it);
    } else {
      ++it;
    }
  }
  auto hi = g_lt_handle.find(std::make_pair(dev, (uintptr_t)s));
  if (hi != g_lt_handle.end()) {
    if (hi->second) ok = hipblasLtDestroy(hi->second) == HIPBLAS_STATUS_SUCCESS && ok;
    g_lt_handle.erase(hi);
  }
  if (!ok) {
    set_error("release_stream_state: a hipBLASLt handle or plan could not be released");
    return IFK_ERR_HIP;
  }
  return IFK_OK;
}

int lib_gemm_plan(hipStream_t s, int64_t M, int64_t N, int64_t K, int adt, int64_t lda,
                  bool akc, int bdt, int64_t ldb, bool bkc, int64_t ldc, bool beta_nz,
                  size_t ws_bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  hipblasLtHandle_t h = nullptr;
  const LtPlan* pl = lt_plan(LtKey{dev, (uintptr_t)s, M, N, K, lda, ldb, ldc, beta_nz ? 1 : 0,
                                   ws_bytes, adt, akc ? 1 : 0, bdt, bkc ? 1 : 0},
                             &h);
  return (pl && pl->ok) ? 1 : 0;
}

int lib_gemm_run(hipStream_t s, int64_t M, int64_t N, int64_t K, float alpha, const void* A,
                 int adt, int64_t lda, bool akc, const void* B, int bdt, int64_t ldb, bool bkc,
                 float beta, float* C, int64_t ldc, void* ws, size_t ws_bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("gemm: no current device");
    return IFK_ERR_HIP;
  }
  hipblasLtHandle_t h = nullptr;
  const LtPlan* pl = lt_plan(LtKey{dev, (uintptr_t)s, M, N, K, lda, ldb, ldc,
                                   beta != 0.0f ? 1 : 0, ws_bytes, adt, akc ? 1 : 0, bdt,
                                   bkc ? 1 : 0},
                             &h);
  if (!pl || !pl->ok) {
    set_error("gemm: hipBLASLt has no algorithm for this product");
    return IFK_ERR_INVALID;
  }
  const hipblasStatus_t st = hipblasLtMatmul(h, pl->desc, &alpha, B, pl->la, A, pl->lb, &beta, C,
                                             pl->lc, C, pl->lc, &pl->algo, ws, ws_bytes, s);
  if (st != HIPBLAS_STATUS_SUCCESS) {
    set_error("gemm: hipblasLtMatmul failed");
    return IFK_ERR_HIP;
  }
  return IFK_OK;
}

}  // namespace ifk
