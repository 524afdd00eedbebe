// Host orchestration of the curvature path.  Every routine enqueues work on
// the given stream, takes all scratch memory from the caller's workspace and
// returns IFK_OK or a negative status with the message in get_error().
#pragma once
#include "common.h"
#include "gemm.h"

namespace ifk {

constexpr int PANEL_B = 64;   // column panel width of the fold
constexpr int TRINV_NB = 64;  // diagonal block of the triangular inverse

// streaming_tsqr_update: R (n x n buffer, rows [0, r_in) valid) absorbs X (p x n).
size_t fold_ws(int64_t p, int64_t n);
int fold(hipStream_t s, const void* X, int xdt, int64_t p, int64_t n, int64_t ldx, float* R,
         int64_t ldr, int64_t r_in, int math, void* ws, size_t ws_bytes, int64_t* r_out);

// finalize_R with the 1/sqrt(rows) scale: out = R_damped of [scale * R_in; sqrt(damping) I].
size_t finalize_ws(int64_t n);
int finalize(hipStream_t s, const float* R_in, int64_t ldr_in, int64_t n, float scale,
             float damping, void* out, int odt, int64_t ldo, int math, int* finite, void* ws,
             size_t ws_bytes);

// finalize(fold(R_in, X)) without the undamped running factor: out = R_damped
// of [scale R_in[0:r_in]; scale X; sqrt(damping) I] by a single TPQRT fold.
size_t fold_finalize_ws(int64_t p, int64_t n, int64_t r_in);
int fold_finalize(hipStream_t s, const void* X, int xdt, int64_t p, int64_t n, int64_t ldx,
                  const float* R_in, int64_t ldr, int64_t r_in, float scale, float damping,
                  void* out, int odt, int64_t ldo, int math, int* finite, void* ws,
                  size_t ws_bytes);

// fold_finalize with each 1024-column outer block factored by CholeskyQR2 +
// Householder reconstruction instead of its 64-column panel chain.  *status:
// 1 finite, 0 not finite, 2 a block was too ill-conditioned for CholeskyQR
// (the output is meaningless; fold_finalize computes it).
size_t fold_finalize_cqr_ws(int64_t p, int64_t n, int64_t r_in);
int fold_finalize_cqr(hipStream_t s, const void* X, int xdt, int64_t p, int64_t n, int64_t ldx,
                      const float* R_in, int64_t ldr, int64_t r_in, float scale, float damping,
                      void* out, int odt, int64_t ldo, int math, int* status, void* ws,
                      size_t ws_bytes);

// The same factor as fold_finalize from the Gram matrix of [R_in; X] and a
// blocked Cholesky (gramchol.hip; bf16 arithmetic only).  *status as for
// fold_finalize_cqr (2: a pivot below pivot_tol of its Gram diagonal).  With
// kappa_bound, an upper bound of kappa_2 of the factor from the Gram
// matrix's Frobenius norm (device float).  batch factors of the same shape
// at once: X and R_in are host arrays of batch device pointers, entry b's
// factor goes to out + b * out_stride, its status to status[b] and its bound
// to kappa_bound[b].
// With inv, also Z = R^{-1} and its RNE bf16 copies Zb = Z (upper) and
// ZTb = Z^T (lower): diagonal GB-blocks from the chain's block inverses (of
// the fp32 factor), the rest by the bf16 block-doubling levels on the output
// factor (fold_finalize_gram_inv_ws workspace); entry b's at the element
// strides sz, sb.
struct GramInverse {
  float* Z;
  int64_t ldz, sz;
  bf16_t *Zb, *ZT;
  int64_t ldb, sb;
};
// The factor update's default relative pivot threshold of the Gram route
// (the streaming fold's caller passes its own).
constexpr float GRAM_PIVOT_TOL = 1e-3f;
// With split_r, R_in enters the Gram matrix as R_in = hi + lo (both RNE
// bf16; R_in^T R_in to about 2^-17 by three products, K = 3 r_in) instead of
// its bf16 rounding: the streaming fold's running factor is fp32 state, and a
// 2^-9 rounding of it at every fold would add up along a stream.
size_t fold_finalize_gram_ws(int64_t batch, int64_t p, int64_t n, int64_t r_in,
                             bool split_r = false);
size_t fold_finalize_gram_inv_ws(int64_t batch, int64_t p, int64_t n, int64_t r_in);
int fold_finalize_gram(hipStream_t s, int64_t batch, const void* const* X, int xdt, int64_t p,
                       int64_t n, int64_t ldx, const float* const* R_in, int64_t ldr,
                       int64_t r_in, float scale, float damping, void* out, int odt, int64_t ldo,
                       int64_t out_stride, int math, int* status, float* kappa_bound, void* ws,
                       size_t ws_bytes, float pivot_tol = GRAM_PIVOT_TOL,
                       const GramInverse* inv = nullptr, bool split_r = false);

// The streaming fold by the Gram route (bf16 arithmetic): R (rows [0, r_in)
// valid) <- the factor of [R[0:r_in]; X] when r_in + p >= n; *status 1 (R
// written) or 2 (a pivot below pivot_tol of its Gram diagonal, or input not
// finite), R unchanged unless 1.  The running factor R enters split (hi + lo
// bf16), the chunk X as its RNE bf16 rounding.
size_t tsqr_fold_gram_ws(int64_t p, int64_t n, int64_t r_in);
int tsqr_fold_gram(hipStream_t s, const void* X, int xdt, int64_t p, int64_t n, int64_t ldx,
                   float* R, int64_t ldr, int64_t r_in, float pivot_tol, int* status, void* ws,
                   size_t ws_bytes);

// The same for B running factors of one shape, each folding its own chunk,
// in one chain of launches (fold_finalize_gram's batch): R[e] and status[e]
// exactly as tsqr_fold_gram gives them for that entry alone.
size_t tsqr_fold_gram_batched_ws(int64_t batch, int64_t p, int64_t n, int64_t r_in);
int tsqr_fold_gram_batched(hipStream_t s, int64_t batch, const void* const* X, int xdt,
                           int64_t p, int64_t n, int64_t ldx, float* const* R, int64_t ldr,
                           int64_t r_in, float pivot_tol, int* status, void* ws,
                           size_t ws_bytes);

// Z = R^{-1} for upper-triangular R (dtype rdt); Z fp32 upper triangular.
size_t trinv_ws(int64_t n);
int trinv(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z, int64_t ldz,
          int math, int safe, void* ws, size_t ws_bytes);

// The block-doubling levels of the bf16-arithmetic triangular inverse from
// width w0 on, Z12 = -Z11 (R12 Z22): Z's (and Zb's, ZT's) diagonal w0-blocks
// are given, the rest of their triangles is formed (tmpT: n^2 / 4 bf16).
int trinv_levels_t(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, int64_t w0,
                   float* Z, int64_t ldz, bf16_t* ZT, bf16_t* Zb, int64_t ldb, bf16_t* tmpT,
                   SplitScratch sp);

// Z = R^{-1} in bf16 arithmetic, plus RNE bf16 copies Zb = Z and ZTb = Z^T
// (row stride ldb, the other triangle zero) for precondition_apply_b.
size_t trinv_copies_ws(int64_t n);
// fp32-accurate inverse on bf16 MFMA (split halves for the wide levels)
size_t trinv_x3_ws(int64_t n, int rdt);
int trinv_x3(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z, int64_t ldz,
             void* ws, size_t ws_bytes);
int trinv_copies(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z,
                 int64_t ldz, bf16_t* Zb, bf16_t* ZTb, int64_t ldb, void* ws, size_t ws_bytes);

// kappa_2 estimate of an upper-triangular R from R and Z = R^{-1} (device
// float out).
size_t cond_est_ws(int64_t n);
int cond_est(hipStream_t s, const void* R, int rdt, int64_t ldr, const float* Z, int64_t ldz,
             int64_t n, float* kappa, void* ws, size_t ws_bytes);

// nat as precondition_apply in bf16 arithmetic, from the copies of
// trinv_copies (nothing to cast but grad).
size_t precondition_apply_b_min_ws(int64_t n_out, int64_t n_in);
int precondition_apply_b_fit(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in,
                             int64_t ldg, const bf16_t* ZXb, const bf16_t* ZXt, int64_t ldx2,
                             const bf16_t* ZGb, const bf16_t* ZGt, int64_t ldg2, float* nat,
                             int64_t ldn, void* ws, size_t ws_bytes);
size_t precondition_apply_b_ws(int64_t n_out, int64_t n_in);
int precondition_apply_b(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in,
                         int64_t ldg, const bf16_t* ZXb, const bf16_t* ZXt, int64_t ldx2,
                         const bf16_t* ZGb, const bf16_t* ZGt, int64_t ldg2, float* nat,
                         int64_t ldn, void* ws, size_t ws_bytes);

// Classic K-FAC control: S = beta S + X^T X (full symmetric, fp32), the damped
// SPD inverse (A + damping I)^{-1} by Cholesky, and nat = G^{-1} grad A^{-1}.
size_t gram_accumulate_ws(int64_t n);
int gram_accumulate(hipStream_t s, const void* X, int xdt, int64_t p, int64_t n, int64_t ldx,
                    float* S, int64_t lds, float beta, void* ws, size_t ws_bytes);
size_t inv_spd_damped_ws(int64_t n);
int inv_spd_damped(hipStream_t s, const void* A, int adt, int64_t n, int64_t lda, float damping,
                   float* X, int64_t ldx, void* ws, size_t ws_bytes);
size_t classic_precondition_ws(int64_t n_out, int64_t n_in);
int classic_precondition(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in,
                         int64_t ldg, const float* A_inv, int64_t ldai, const float* G_inv,
                         int64_t ldgi, float* nat, int64_t ldn, void* ws, size_t ws_bytes);

// Laplace consumer: R^T R = V diag(eig) V^T from R (one-sided block Jacobi SVD
// of R, eig = sigma^2 descending, *sweeps = sweeps to convergence, negative if
// not converged); the posterior scales 1 / sqrt(sqrt_n d + sqrt_lam); one
// weight sample W = W_map + U_G diag(s_G) Xi diag(s_A) U_A^T.
size_t factor_evd_ws(int64_t n);
int factor_evd(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* V,
               int64_t ldv, float* eig, int* sweeps, void* ws, size_t ws_bytes);
int laplace_scales(hipStream_t s, const float* d, int64_t n, float sqrt_n, float sqrt_lam,
                   float* out);
size_t laplace_sample_ws(int64_t n_out, int64_t n_in);
int laplace_sample(hipStream_t s, const float* W_map, int64_t ldm, float* W, int64_t ldw,
                   int64_t n_out, int64_t n_in, const float* U_G, int64_t ldug, const float* s_G,
                   const float* U_A, int64_t ldua, const float* s_A, const float* Xi,
                   int64_t ldxi, void* ws, size_t ws_bytes);

// bf16 halves of an fp32 inverse for precondition_apply_x3: Z = Zh + Zl and
// Z^T = ZTh + ZTl (row stride ldb).
int split_inverse(hipStream_t s, const float* Z, int64_t ldz, int64_t n, bf16_t* Zh, bf16_t* Zl,
                  bf16_t* ZTh, bf16_t* ZTl, int64_t ldb);
// nat = Z_G Z_G^T grad Z_X Z_X^T at fp32 accuracy from split bf16 operands:
// ZX, ZG = {Z_hi, Z_lo, Z^T_hi, Z^T_lo}, row strides ldx, ldg2.
size_t precondition_apply_x3_ws(int64_t n_out, int64_t n_in);
int precondition_apply_x3(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in,
                          int64_t ldg, const bf16_t* const* ZX, int64_t ldx,
                          const bf16_t* const* ZG, int64_t ldg2, float* nat, int64_t ldn, void* ws,
                          size_t ws_bytes);

// The two applies for B layers of one shape in grouped launches: each
// product is one launch over the batch, every entry getting the bits the
// single-layer call gives it.  Inverse copies (and their halves) sit at a
// fixed element stride from entry to entry (sx, sg), the results at snat; the
// gradients are given by pointer (ldg each).
size_t precondition_apply_b_batched_ws(int64_t batch, int64_t n_out, int64_t n_in);
int precondition_apply_b_batched(hipStream_t s, int64_t batch, const float* const* grad,
                                 int64_t n_out, int64_t n_in, int64_t ldg, const bf16_t* ZXb,
                                 const bf16_t* ZXt, int64_t ldx2, int64_t sx, const bf16_t* ZGb,
                                 const bf16_t* ZGt, int64_t ldg2, int64_t sg, float* nat,
                                 int64_t ldn, int64_t snat, void* ws, size_t ws_bytes);
size_t precondition_apply_x3_batched_ws(int64_t batch, int64_t n_out, int64_t n_in);
int precondition_apply_x3_batched(hipStream_t s, int64_t batch, const float* const* grad,
                                  int64_t n_out, int64_t n_in, int64_t ldg,
                                  const bf16_t* const* ZX, int64_t ldx, int64_t sx,
                                  const bf16_t* const* ZG, int64_t ldg2, int64_t sg, float* nat,
                                  int64_t ldn, int64_t snat, void* ws, size_t ws_bytes);

// nat = Z_G Z_G^T grad Z_X Z_X^T, with Z_X = R_X^{-1}, Z_G = R_G^{-1} given.
size_t precondition_apply_ws(int64_t n_out, int64_t n_in, int math);
int precondition_apply(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in, int64_t ldg,
                       const float* ZX, int64_t ldzx, const float* ZG, int64_t ldzg, float* nat,
                       int64_t ldn, int math, void* ws, size_t ws_bytes);

// All four solves from the factors themselves (inverses formed internally).
size_t precondition_ws(int64_t n_out, int64_t n_in, int math);
int precondition(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in, int64_t ldg,
                 const void* RX, int64_t ldrx, const void* RG, int64_t ldrg, int rdt, float* nat,
                 int64_t ldn, int math, void* ws, size_t ws_bytes);

// out = Z_G Z_G^T g for a bias gradient g (n_out).
size_t precondition_bias_ws(int64_t n_out);
int precondition_bias(hipStream_t s, const float* g, int64_t n_out, const float* ZG, int64_t ldzg,
                      float* out, void* ws, size_t ws_bytes);

// bf16_linalg counterparts ------------------------------------------------------
size_t geqrf_r_ws(int64_t m, int64_t n);
int geqrf_r(hipStream_t s, const void* A, int adt, int64_t m, int64_t n, int64_t lda, void* R,
            int rdt, int64_t ldr, int math, void* ws, size_t ws_bytes);

size_t trsm_ws(int64_t n, int64_t k);
int trsm(hipStream_t s, const void* R, int rdt, int64_t n, int64_t ldr, int upper, const void* B,
         int bdt, int64_t k, int64_t ldb, void* X, int xdt, int64_t ldx, int math, void* ws,
         size_t ws_bytes);

size_t potrf_ws(int64_t n);
int potrf(hipStream_t s, const void* A, int adt, int64_t n, int64_t lda, void* L, int ldt,
          int64_t ldl, int math, void* ws, size_t ws_bytes);

size_t inv_spd_ws(int64_t n);
int inv_spd(hipStream_t s, const void* A, int adt, int64_t n, int64_t lda, void* X, int xdt,
            int64_t ldx, int math, void* ws, size_t ws_bytes);

}  // namespace ifk
