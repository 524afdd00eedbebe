// extern "C" entry points declared in include/ifkfac_hip.h.  Each validates
// what the kernels assume about shapes before anything is launched, and maps
// every failure to a status code plus a thread-local message.
#include "../../include/ifkfac_hip.h"

#include <algorithm>
#include <string>

#include "gemm.h"
#include "kernels.h"
#include "linalg.h"
#include "lookahead.h"

namespace ifk {

static thread_local std::string g_err;

void set_error(const std::string& msg) { g_err = msg; }
const char* get_error() { return g_err.c_str(); }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_err = std::string(what) + ": " + hipGetErrorString(e);
    return IFK_ERR_HIP;
  }
  return IFK_OK;
}

static bool dt_ok(int dt) { return dt == DT_F32 || dt == DT_BF16; }
static bool math_ok(int m) { return m == MATH_F32 || m == MATH_BF16; }

}  // namespace ifk

using namespace ifk;

#define GUARD(cond, msg)            \
  do {                              \
    if (!(cond)) {                  \
      set_error(msg);               \
      return IFK_ERR_INVALID;       \
    }                               \
  } while (0)

extern "C" {

int ifk_abi_version(void) { return 2; }

const char* ifk_last_error(void) { return get_error(); }

size_t ifk_tsqr_fold_workspace_size(int64_t p, int64_t n) {
  if (p < 0 || n < 1) return 0;
  return fold_ws(p, n);
}

int ifk_tsqr_fold(void* stream, const void* X, int x_dtype, int64_t p, int64_t n, int64_t ldx,
                  float* R, int64_t ldr, int64_t r_in, int math, void* workspace,
                  size_t workspace_bytes, int64_t* r_out) {
  GUARD(dt_ok(x_dtype) && math_ok(math), "tsqr_fold: bad dtype or math code");
  return fold((hipStream_t)stream, X, x_dtype, p, n, ldx, R, ldr, r_in, math, workspace,
              workspace_bytes, r_out);
}

size_t ifk_finalize_workspace_size(int64_t n) {
  if (n < 1) return 0;
  return finalize_ws(n);
}

int ifk_finalize(void* stream, const float* R_in, int64_t ldr_in, int64_t n, float scale,
                 float damping, void* out, int out_dtype, int64_t ldo, int math, int32_t* finite,
                 void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(out_dtype) && math_ok(math), "finalize: bad dtype or math code");
  return finalize((hipStream_t)stream, R_in, ldr_in, n, scale, damping, out, out_dtype, ldo, math,
                  finite, workspace, workspace_bytes);
}

size_t ifk_fold_finalize_workspace_size(int64_t p, int64_t n, int64_t r_in) {
  if (p < 0 || n < 1 || r_in < 0 || r_in > n) return 0;
  return fold_finalize_ws(p, n, r_in);
}

int ifk_fold_finalize(void* stream, const void* X, int x_dtype, int64_t p, int64_t n,
                      int64_t ldx, const float* R_in, int64_t ldr, int64_t r_in, float scale,
                      float damping, void* out, int out_dtype, int64_t ldo, int math,
                      int32_t* finite, void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(x_dtype) && dt_ok(out_dtype) && math_ok(math),
        "fold_finalize: bad dtype or math code");
  return fold_finalize((hipStream_t)stream, X, x_dtype, p, n, ldx, R_in, ldr, r_in, scale,
                       damping, out, out_dtype, ldo, math, finite, workspace, workspace_bytes);
}

size_t ifk_fold_finalize_cqr_workspace_size(int64_t p, int64_t n, int64_t r_in) {
  if (p < 0 || n < 1 || r_in < 0 || r_in > n) return 0;
  return fold_finalize_cqr_ws(p, n, r_in);
}

int ifk_fold_finalize_cqr(void* stream, const void* X, int x_dtype, int64_t p, int64_t n,
                          int64_t ldx, const float* R_in, int64_t ldr, int64_t r_in, float scale,
                          float damping, void* out, int out_dtype, int64_t ldo, int math,
                          int32_t* status, void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(x_dtype) && dt_ok(out_dtype) && math_ok(math),
        "fold_finalize_cqr: bad dtype or math code");
  return fold_finalize_cqr((hipStream_t)stream, X, x_dtype, p, n, ldx, R_in, ldr, r_in, scale,
                           damping, out, out_dtype, ldo, math, status, workspace,
                           workspace_bytes);
}

size_t ifk_fold_finalize_gram_workspace_size(int64_t p, int64_t n, int64_t r_in) {
  if (p < 0 || n < 1 || r_in < 0 || r_in > n) return 0;
  return fold_finalize_gram_ws(1, p, n, r_in);
}

int ifk_fold_finalize_gram(void* stream, const void* X, int x_dtype, int64_t p, int64_t n,
                           int64_t ldx, const float* R_in, int64_t ldr, int64_t r_in, float scale,
                           float damping, void* out, int out_dtype, int64_t ldo, int math,
                           int32_t* status, float* kappa_bound, void* workspace,
                           size_t workspace_bytes) {
  GUARD(dt_ok(x_dtype) && dt_ok(out_dtype) && math_ok(math),
        "fold_finalize_gram: bad dtype or math code");
  const void* xs[1] = {X};
  const float* rs[1] = {R_in};
  return fold_finalize_gram((hipStream_t)stream, 1, xs, x_dtype, p, n, ldx, rs, ldr, r_in, scale,
                            damping, out, out_dtype, ldo, n * ldo, math, status, kappa_bound,
                            workspace, workspace_bytes);
}

size_t ifk_tsqr_fold_gram_workspace_size(int64_t p, int64_t n, int64_t r_in) {
  if (p < 0 || n < 1 || r_in < 0 || r_in > n) return 0;
  return tsqr_fold_gram_ws(p, n, r_in);
}

int ifk_tsqr_fold_gram(void* stream, const void* X, int x_dtype, int64_t p, int64_t n,
                       int64_t ldx, float* R, int64_t ldr, int64_t r_in, float pivot_tol,
                       int32_t* status, void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(x_dtype), "tsqr_fold_gram: bad dtype");
  return tsqr_fold_gram((hipStream_t)stream, X, x_dtype, p, n, ldx, R, ldr, r_in, pivot_tol,
                        status, workspace, workspace_bytes);
}

size_t ifk_tsqr_fold_gram_batched_workspace_size(int64_t batch, int64_t p, int64_t n,
                                                  int64_t r_in) {
  if (batch < 1 || p < 0 || n < 1 || r_in < 0 || r_in > n) return 0;
  return tsqr_fold_gram_batched_ws(batch, p, n, r_in);
}

int ifk_tsqr_fold_gram_batched(void* stream, int64_t batch, const void* const* X, int x_dtype,
                               int64_t p, int64_t n, int64_t ldx, float* const* R, int64_t ldr,
                               int64_t r_in, float pivot_tol, int32_t* status, void* workspace,
                               size_t workspace_bytes) {
  GUARD(dt_ok(x_dtype), "tsqr_fold_gram_batched: bad dtype");
  return tsqr_fold_gram_batched((hipStream_t)stream, batch, X, x_dtype, p, n, ldx, R, ldr, r_in,
                                pivot_tol, status, workspace, workspace_bytes);
}

size_t ifk_fold_finalize_gram_batched_workspace_size(int64_t batch, int64_t p, int64_t n,
                                                     int64_t r_in) {
  if (batch < 1 || p < 0 || n < 1 || r_in < 0 || r_in > n) return 0;
  return fold_finalize_gram_ws(batch, p, n, r_in);
}

int ifk_fold_finalize_gram_batched(void* stream, int64_t batch, const void* const* X, int x_dtype,
                                   int64_t p, int64_t n, int64_t ldx, const float* const* R_in,
                                   int64_t ldr, int64_t r_in, float scale, float damping,
                                   void* out, int out_dtype, int64_t ldo, int64_t out_stride,
                                   int math, float pivot_tol, int32_t* status, float* kappa_bound,
                                   void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(x_dtype) && dt_ok(out_dtype) && math_ok(math),
        "fold_finalize_gram_batched: bad dtype or math code");
  return fold_finalize_gram((hipStream_t)stream, batch, X, x_dtype, p, n, ldx, R_in, ldr, r_in,
                            scale, damping, out, out_dtype, ldo, out_stride, math, status,
                            kappa_bound, workspace, workspace_bytes, pivot_tol);
}

size_t ifk_fold_finalize_gram_inverse_workspace_size(int64_t batch, int64_t p, int64_t n,
                                                     int64_t r_in) {
  if (batch < 1 || p < 0 || n < 1 || r_in < 0 || r_in > n) return 0;
  return fold_finalize_gram_inv_ws(batch, p, n, r_in);
}

int ifk_fold_finalize_gram_inverse(void* stream, int64_t batch, const void* const* X, int x_dtype,
                                   int64_t p, int64_t n, int64_t ldx, const float* const* R_in,
                                   int64_t ldr, int64_t r_in, float scale, float damping,
                                   void* out, int out_dtype, int64_t ldo, int64_t out_stride,
                                   float pivot_tol, int32_t* status, float* kappa_bound, float* Z,
                                   int64_t ldz, int64_t z_stride, void* Zb, void* ZTb, int64_t ldb,
                                   int64_t b_stride, void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(x_dtype) && dt_ok(out_dtype), "fold_finalize_gram_inverse: bad dtype");
  GramInverse inv{Z, ldz, z_stride, (bf16_t*)Zb, (bf16_t*)ZTb, ldb, b_stride};
  return fold_finalize_gram((hipStream_t)stream, batch, X, x_dtype, p, n, ldx, R_in, ldr, r_in,
                            scale, damping, out, out_dtype, ldo, out_stride, MATH_BF16, status,
                            kappa_bound, workspace, workspace_bytes, pivot_tol, &inv);
}

int ifk_status_to_host(void* stream, const int32_t* status, int32_t* host_status, int64_t n) {
  if (n < 1 || n > (1 << 20) || !status || !host_status) {
    set_error("status_to_host: invalid arguments");
    return IFK_ERR_INVALID;
  }
  void* dev = nullptr;
  if (hipHostGetDevicePointer(&dev, host_status, 0) != hipSuccess || !dev) {
    (void)hipGetLastError();
    set_error("status_to_host: host_status is not pinned host memory (hipHostMalloc)");
    return IFK_ERR_INVALID;
  }
  return launch_status_to_host((hipStream_t)stream, status, (int*)dev, (int)n);
}

int ifk_release_stream_state(void* stream) {
  return look_ahead_release((hipStream_t)stream);
}

size_t ifk_tri_inverse_workspace_size(int64_t n) {
  if (n < 1) return 0;
  return trinv_ws(n);
}

int ifk_tri_inverse(void* stream, const void* R, int r_dtype, int64_t ldr, int64_t n, float* Z,
                    int64_t ldz, int math, void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(r_dtype) && math_ok(math), "tri_inverse: bad dtype or math code");
  return trinv((hipStream_t)stream, R, r_dtype, ldr, n, Z, ldz, math, 0, workspace,
               workspace_bytes);
}

size_t ifk_tri_inverse_bf16_workspace_size(int64_t n) {
  if (n < 1) return 0;
  return trinv_copies_ws(n);
}

int ifk_tri_inverse_bf16(void* stream, const void* R, int r_dtype, int64_t ldr, int64_t n,
                         float* Z, int64_t ldz, void* Zb, void* ZTb, int64_t ldb, void* workspace,
                         size_t workspace_bytes) {
  GUARD(dt_ok(r_dtype), "tri_inverse_bf16: bad dtype code");
  return trinv_copies((hipStream_t)stream, R, r_dtype, ldr, n, Z, ldz, (bf16_t*)Zb, (bf16_t*)ZTb,
                      ldb, workspace, workspace_bytes);
}

size_t ifk_tri_inverse_x3_workspace_size(int64_t n, int r_dtype) {
  if (n < 1 || !dt_ok(r_dtype)) return 0;
  return trinv_x3_ws(n, r_dtype);
}

int ifk_tri_inverse_x3(void* stream, const void* R, int r_dtype, int64_t ldr, int64_t n, float* Z,
                       int64_t ldz, void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(r_dtype), "tri_inverse_x3: bad dtype code");
  return trinv_x3((hipStream_t)stream, R, r_dtype, ldr, n, Z, ldz, workspace, workspace_bytes);
}

size_t ifk_cond_estimate_workspace_size(int64_t n) {
  if (n < 1) return 0;
  return cond_est_ws(n);
}

int ifk_cond_estimate(void* stream, const void* R, int r_dtype, int64_t ldr, const float* Z,
                      int64_t ldz, int64_t n, float* kappa, void* workspace,
                      size_t workspace_bytes) {
  GUARD(dt_ok(r_dtype), "cond_estimate: bad dtype code");
  return cond_est((hipStream_t)stream, R, r_dtype, ldr, Z, ldz, n, kappa, workspace,
                  workspace_bytes);
}

size_t ifk_precondition_apply_bf16_workspace_size(int64_t n_out, int64_t n_in) {
  if (n_out < 1 || n_in < 1) return 0;
  return precondition_apply_b_ws(n_out, n_in);
}

int ifk_precondition_apply_bf16(void* stream, const float* grad, int64_t n_out, int64_t n_in,
                                int64_t ldg, const void* Z_Xb, const void* Z_Xt, int64_t ldzx,
                                const void* Z_Gb, const void* Z_Gt, int64_t ldzg, float* nat,
                                int64_t ldn, void* workspace, size_t workspace_bytes) {
  return precondition_apply_b((hipStream_t)stream, grad, n_out, n_in, ldg, (const bf16_t*)Z_Xb,
                              (const bf16_t*)Z_Xt, ldzx, (const bf16_t*)Z_Gb, (const bf16_t*)Z_Gt,
                              ldzg, nat, ldn, workspace, workspace_bytes);
}

int ifk_inverse_split_copies(void* stream, const float* Z, int64_t ldz, int64_t n, void* Z_hi,
                             void* Z_lo, void* ZT_hi, void* ZT_lo, int64_t ldb) {
  return split_inverse((hipStream_t)stream, Z, ldz, n, (bf16_t*)Z_hi, (bf16_t*)Z_lo,
                       (bf16_t*)ZT_hi, (bf16_t*)ZT_lo, ldb);
}

size_t ifk_precondition_apply_x3_workspace_size(int64_t n_out, int64_t n_in) {
  if (n_out < 1 || n_in < 1) return 0;
  return precondition_apply_x3_ws(n_out, n_in);
}

int ifk_precondition_apply_x3(void* stream, const float* grad, int64_t n_out, int64_t n_in,
                              int64_t ldg, const void* Z_X_hi, const void* Z_X_lo,
                              const void* Z_XT_hi, const void* Z_XT_lo, int64_t ldzx,
                              const void* Z_G_hi, const void* Z_G_lo, const void* Z_GT_hi,
                              const void* Z_GT_lo, int64_t ldzg, float* nat, int64_t ldn,
                              void* workspace, size_t workspace_bytes) {
  const bf16_t* zx[4] = {(const bf16_t*)Z_X_hi, (const bf16_t*)Z_X_lo, (const bf16_t*)Z_XT_hi,
                         (const bf16_t*)Z_XT_lo};
  const bf16_t* zg[4] = {(const bf16_t*)Z_G_hi, (const bf16_t*)Z_G_lo, (const bf16_t*)Z_GT_hi,
                         (const bf16_t*)Z_GT_lo};
  return precondition_apply_x3((hipStream_t)stream, grad, n_out, n_in, ldg, zx, ldzx, zg, ldzg, nat,
                               ldn, workspace, workspace_bytes);
}

size_t ifk_precondition_apply_bf16_batched_workspace_size(int64_t batch, int64_t n_out,
                                                          int64_t n_in) {
  if (batch < 1 || n_out < 1 || n_in < 1) return 0;
  return precondition_apply_b_batched_ws(batch, n_out, n_in);
}

int ifk_precondition_apply_bf16_batched(void* stream, int64_t batch, const float* const* grad,
                                        int64_t n_out, int64_t n_in, int64_t ldg,
                                        const void* Z_Xb, const void* Z_Xt, int64_t ldzx,
                                        int64_t stride_zx, const void* Z_Gb, const void* Z_Gt,
                                        int64_t ldzg, int64_t stride_zg, float* nat, int64_t ldn,
                                        int64_t stride_nat, void* workspace,
                                        size_t workspace_bytes) {
  return precondition_apply_b_batched((hipStream_t)stream, batch, grad, n_out, n_in, ldg,
                                      (const bf16_t*)Z_Xb, (const bf16_t*)Z_Xt, ldzx, stride_zx,
                                      (const bf16_t*)Z_Gb, (const bf16_t*)Z_Gt, ldzg, stride_zg,
                                      nat, ldn, stride_nat, workspace, workspace_bytes);
}

size_t ifk_precondition_apply_x3_batched_workspace_size(int64_t batch, int64_t n_out,
                                                        int64_t n_in) {
  if (batch < 1 || n_out < 1 || n_in < 1) return 0;
  return precondition_apply_x3_batched_ws(batch, n_out, n_in);
}

int ifk_precondition_apply_x3_batched(void* stream, int64_t batch, const float* const* grad,
                                      int64_t n_out, int64_t n_in, int64_t ldg,
                                      const void* Z_X_hi, const void* Z_X_lo, const void* Z_XT_hi,
                                      const void* Z_XT_lo, int64_t ldzx, int64_t stride_zx,
                                      const void* Z_G_hi, const void* Z_G_lo, const void* Z_GT_hi,
                                      const void* Z_GT_lo, int64_t ldzg, int64_t stride_zg,
                                      float* nat, int64_t ldn, int64_t stride_nat,
                                      void* workspace, size_t workspace_bytes) {
  const bf16_t* zx[4] = {(const bf16_t*)Z_X_hi, (const bf16_t*)Z_X_lo, (const bf16_t*)Z_XT_hi,
                         (const bf16_t*)Z_XT_lo};
  const bf16_t* zg[4] = {(const bf16_t*)Z_G_hi, (const bf16_t*)Z_G_lo, (const bf16_t*)Z_GT_hi,
                         (const bf16_t*)Z_GT_lo};
  return precondition_apply_x3_batched((hipStream_t)stream, batch, grad, n_out, n_in, ldg, zx,
                                       ldzx, stride_zx, zg, ldzg, stride_zg, nat, ldn, stride_nat,
                                       workspace, workspace_bytes);
}

size_t ifk_precondition_workspace_size(int64_t n_out, int64_t n_in, int math) {
  if (n_out < 1 || n_in < 1 || !math_ok(math)) return 0;
  return precondition_ws(n_out, n_in, math);
}

int ifk_precondition(void* stream, const float* grad, int64_t n_out, int64_t n_in, int64_t ldg,
                     const void* R_X, int64_t ldrx, const void* R_G, int64_t ldrg, int r_dtype,
                     float* nat, int64_t ldn, int math, void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(r_dtype) && math_ok(math), "precondition: bad dtype or math code");
  return precondition((hipStream_t)stream, grad, n_out, n_in, ldg, R_X, ldrx, R_G, ldrg, r_dtype,
                      nat, ldn, math, workspace, workspace_bytes);
}

size_t ifk_precondition_apply_workspace_size(int64_t n_out, int64_t n_in, int math) {
  if (n_out < 1 || n_in < 1 || !math_ok(math)) return 0;
  return precondition_apply_ws(n_out, n_in, math);
}

int ifk_precondition_apply(void* stream, const float* grad, int64_t n_out, int64_t n_in,
                           int64_t ldg, const float* Z_X, int64_t ldzx, const float* Z_G,
                           int64_t ldzg, float* nat, int64_t ldn, int math, void* workspace,
                           size_t workspace_bytes) {
  GUARD(math_ok(math), "precondition_apply: bad math code");
  return precondition_apply((hipStream_t)stream, grad, n_out, n_in, ldg, Z_X, ldzx, Z_G, ldzg, nat,
                            ldn, math, workspace, workspace_bytes);
}

size_t ifk_precondition_bias_workspace_size(int64_t n_out) {
  if (n_out < 1) return 0;
  return precondition_bias_ws(n_out);
}

int ifk_precondition_bias(void* stream, const float* g, int64_t n_out, const float* Z_G,
                          int64_t ldzg, float* out, void* workspace, size_t workspace_bytes) {
  return precondition_bias((hipStream_t)stream, g, n_out, Z_G, ldzg, out, workspace,
                           workspace_bytes);
}

int ifk_momentum_update(void* stream, const float* nat, float* buf, float* W, int64_t numel,
                        float lr, float momentum, float weight_decay, int buf_init) {
  GUARD(numel >= 0, "momentum_update: negative size");
  GUARD(numel == 0 || (nat && W), "momentum_update: null pointer");
  return launch_momentum_update((hipStream_t)stream, nat, buf, W, numel, lr, momentum,
                                weight_decay, buf_init);
}

size_t ifk_geqrf_r_workspace_size(int64_t m, int64_t n) {
  if (m < n || n < 1) return 0;
  return geqrf_r_ws(m, n);
}

int ifk_geqrf_r(void* stream, const void* A, int a_dtype, int64_t m, int64_t n, int64_t lda,
                void* R, int r_dtype, int64_t ldr, int math, void* workspace,
                size_t workspace_bytes) {
  GUARD(dt_ok(a_dtype) && dt_ok(r_dtype) && math_ok(math), "geqrf_r: bad dtype or math code");
  return geqrf_r((hipStream_t)stream, A, a_dtype, m, n, lda, R, r_dtype, ldr, math, workspace,
                 workspace_bytes);
}

size_t ifk_trsm_workspace_size(int64_t n, int64_t k) {
  if (n < 1 || k < 0) return 0;
  return trsm_ws(n, k);
}

int ifk_trsm(void* stream, const void* R, int r_dtype, int64_t n, int64_t ldr, int upper,
             const void* B, int b_dtype, int64_t k, int64_t ldb, void* X, int x_dtype, int64_t ldx,
             int math, void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(r_dtype) && dt_ok(b_dtype) && dt_ok(x_dtype) && math_ok(math),
        "trsm: bad dtype or math code");
  return trsm((hipStream_t)stream, R, r_dtype, n, ldr, upper, B, b_dtype, k, ldb, X, x_dtype, ldx,
              math, workspace, workspace_bytes);
}

size_t ifk_potrf_workspace_size(int64_t n) {
  if (n < 1) return 0;
  return potrf_ws(n);
}

int ifk_potrf(void* stream, const void* A, int a_dtype, int64_t n, int64_t lda, void* L,
              int l_dtype, int64_t ldl, int math, void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(a_dtype) && dt_ok(l_dtype) && math_ok(math), "potrf: bad dtype or math code");
  return potrf((hipStream_t)stream, A, a_dtype, n, lda, L, l_dtype, ldl, math, workspace,
               workspace_bytes);
}

size_t ifk_inv_spd_workspace_size(int64_t n) {
  if (n < 1) return 0;
  return inv_spd_ws(n);
}

int ifk_inv_spd(void* stream, const void* A, int a_dtype, int64_t n, int64_t lda, void* X,
                int x_dtype, int64_t ldx, int math, void* workspace, size_t workspace_bytes) {
  GUARD(dt_ok(a_dtype) && dt_ok(x_dtype) && math_ok(math), "inv_spd: bad dtype or math code");
  return inv_spd((hipStream_t)stream, A, a_dtype, n, lda, X, x_dtype, ldx, math, workspace,
                 workspace_bytes);
}

size_t ifk_gram_accumulate_workspace_size(int64_t n) {
  if (n < 1) return 0;
  return gram_accumulate_ws(n);
}

int ifk_gram_accumulate(void* stream, const void* X, int x_dtype, int64_t p, int64_t n,
                        int64_t ldx, float* S, int64_t lds, float beta, void* workspace,
                        size_t workspace_bytes) {
  GUARD(dt_ok(x_dtype), "gram_accumulate: bad dtype");
  return gram_accumulate((hipStream_t)stream, X, x_dtype, p, n, ldx, S, lds, beta, workspace,
                         workspace_bytes);
}

int ifk_axpby(void* stream, float alpha, const float* X, int64_t ldx, float beta, float* Y,
              int64_t ldy, int64_t rows, int64_t cols) {
  GUARD(rows >= 0 && cols >= 0 && ldx >= cols && ldy >= cols && (rows * cols == 0 || (X && Y)),
        "axpby: invalid arguments");
  return launch_axpby((hipStream_t)stream, alpha, X, ldx, beta, Y, ldy, rows, cols);
}

size_t ifk_inv_spd_damped_workspace_size(int64_t n) {
  if (n < 1) return 0;
  return inv_spd_damped_ws(n);
}

int ifk_inv_spd_damped(void* stream, const void* A, int a_dtype, int64_t n, int64_t lda,
                       float damping, float* X, int64_t ldx, void* workspace,
                       size_t workspace_bytes) {
  GUARD(dt_ok(a_dtype), "inv_spd_damped: bad dtype");
  return inv_spd_damped((hipStream_t)stream, A, a_dtype, n, lda, damping, X, ldx, workspace,
                        workspace_bytes);
}

size_t ifk_classic_precondition_workspace_size(int64_t n_out, int64_t n_in) {
  if (n_out < 1 || n_in < 1) return 0;
  return classic_precondition_ws(n_out, n_in);
}

int ifk_classic_precondition(void* stream, const float* grad, int64_t n_out, int64_t n_in,
                             int64_t ldg, const float* A_inv, int64_t ldai, const float* G_inv,
                             int64_t ldgi, float* nat, int64_t ldn, void* workspace,
                             size_t workspace_bytes) {
  return classic_precondition((hipStream_t)stream, grad, n_out, n_in, ldg, A_inv, ldai, G_inv,
                              ldgi, nat, ldn, workspace, workspace_bytes);
}

size_t ifk_factor_evd_workspace_size(int64_t n) {
  if (n < 1) return 0;
  return factor_evd_ws(n);
}

int ifk_factor_evd(void* stream, const void* R, int r_dtype, int64_t ldr, int64_t n, float* V,
                   int64_t ldv, float* eigvals, int* sweeps, void* workspace,
                   size_t workspace_bytes) {
  GUARD(dt_ok(r_dtype), "factor_evd: bad dtype");
  return factor_evd((hipStream_t)stream, R, r_dtype, ldr, n, V, ldv, eigvals, sweeps, workspace,
                    workspace_bytes);
}

int ifk_laplace_scales(void* stream, const float* d, int64_t n, float sqrt_n, float sqrt_lam,
                       float* out) {
  return laplace_scales((hipStream_t)stream, d, n, sqrt_n, sqrt_lam, out);
}

size_t ifk_laplace_sample_workspace_size(int64_t n_out, int64_t n_in) {
  if (n_out < 1 || n_in < 1) return 0;
  return laplace_sample_ws(n_out, n_in);
}

int ifk_laplace_sample(void* stream, const float* W_map, int64_t ldm, float* W, int64_t ldw,
                       int64_t n_out, int64_t n_in, const float* U_G, int64_t ldug,
                       const float* s_G, const float* U_A, int64_t ldua, const float* s_A,
                       const float* Xi, int64_t ldxi, void* workspace, size_t workspace_bytes) {
  return laplace_sample((hipStream_t)stream, W_map, ldm, W, ldw, n_out, n_in, U_G, ldug, s_G, U_A,
                        ldua, s_A, Xi, ldxi, workspace, workspace_bytes);
}

size_t ifk_gemm_workspace_size(int64_t m, int64_t n) {
  if (m < 1 || n < 1) return 0;
  size_t f = (size_t)m * n * 64;
  if (f > ((size_t)16 << 20)) f = (size_t)16 << 20;
  // and the stream-K partial tiles of a product with K up to 2^20
  f = std::max(f, gemm_scratch_floats(m, n, (int64_t)1 << 20, 1));
  return f * sizeof(float);
}

int ifk_gemm(void* stream, int math, int64_t m, int64_t n, int64_t k, float alpha, const void* A,
             int a_dtype, int64_t lda, int trans_a, const void* B, int b_dtype, int64_t ldb,
             int trans_b, float beta, float* C, int64_t ldc, void* workspace,
             size_t workspace_bytes) {
  GUARD(dt_ok(a_dtype) && dt_ok(b_dtype) && math_ok(math), "gemm: bad dtype or math code");
  GUARD(m >= 0 && n >= 0 && k >= 0, "gemm: negative size");
  GUARD(trans_a >= 0 && trans_a < 6 && trans_b >= 0 && trans_b < 6,
        "gemm: trans flags out of range");
  const bool ta = trans_a & 1, tb = trans_b & 1;
  const int tra = trans_a >> 1, trb = trans_b >> 1;   // 0 none, 1 upper, 2 lower
  GUARD((tra == 0 || m == k) && (trb == 0 || k == n), "gemm: triangular operand not square");
  GUARD(ldc >= n && (ta ? lda >= m : lda >= k) && (tb ? ldb >= k : ldb >= n),
        "gemm: leading dimension too small");
  GUARD((m == 0 || n == 0) || (C && (k == 0 || (A && B))), "gemm: null pointer");
  const int tri_code[3] = {TRI_NONE, TRI_UPPER, TRI_LOWER};
  const MatRef a = ta ? A_t(A, a_dtype, lda, tri_code[tra]) : A_n(A, a_dtype, lda, tri_code[tra]);
  const MatRef b = tb ? B_t(B, b_dtype, ldb, tri_code[trb]) : B_n(B, b_dtype, ldb, tri_code[trb]);
  SplitScratch sp{(float*)workspace, workspace ? workspace_bytes / sizeof(float) : 0};
  return gemm((hipStream_t)stream, math, m, n, k, alpha, a, b, beta, out_f32(C, ldc), 1, sp);
}

int ifk_profile_begin(int variant) { return profile_begin(variant); }

int ifk_profile_end(int64_t* n_launches) { return profile_end(n_launches); }

int ifk_profile_get(int64_t i, int* variant, float* ms, double* flops, double* bytes, int64_t* m,
                    int64_t* n, int64_t* k) {
  GUARD(variant && ms && flops && bytes && m && n && k, "profile_get: null pointer");
  return profile_get(i, variant, ms, flops, bytes, m, n, k);
}

}  // extern "C"
