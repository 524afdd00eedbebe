/*
 * ifkfac_hip.h -- C ABI of the MI355X (gfx950) IFKFAC curvature library.
 *
 * The library implements, as hand-written HIP kernels, the numerical seams of
 * the reference package (Gsend/ifkfac) that its Python optimizer calls on the
 * curvature hot path.  Each entry point below names the reference function it
 * replaces (file:line in the reference tree).
 *
 * Conventions shared by every entry point
 *   - Matrices are row-major.  `ld*` is the leading dimension in elements.
 *   - Pointers are device pointers (HBM); the library never allocates device
 *     memory and never frees caller memory.  Scratch space comes from the
 *     caller through (workspace, workspace_bytes); the matching
 *     *_workspace_size() function returns how many bytes a call needs.
 *   - `stream` is a hipStream_t.  All work is enqueued on it; no entry point
 *     synchronises the device or the stream.
 *   - Return value: IFK_OK (0) or a negative IFK_ERR_* code.  The message of
 *     the last failure on the calling thread is available from
 *     ifk_last_error().  Nothing throws across this boundary.
 *   - dtype codes: IFK_F32, IFK_BF16.  math codes: IFK_MATH_F32 runs the
 *     contractions on fp32 MFMA; IFK_MATH_BF16 rounds operands to bf16 (RNE)
 *     and runs bf16 MFMA, always with fp32 accumulation.
 */
#ifndef IFKFAC_HIP_H
#define IFKFAC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IFK_OK 0
#define IFK_ERR_INVALID (-1)
#define IFK_ERR_WORKSPACE (-2)
#define IFK_ERR_HIP (-3)

#define IFK_F32 0
#define IFK_BF16 1

#define IFK_MATH_F32 0
#define IFK_MATH_BF16 1

/* Version of this ABI (bumped on any signature change). */
int ifk_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* ifk_last_error(void);

/*
 * Release the helper streams and events that the factorisations of more than
 * 1024 columns create for (current device, calling stream) on first use and
 * otherwise keep until the process ends.  No counterpart in the
 * reference (torch manages its own streams): it is for callers that create
 * many calling streams over a process's life.  Waits for the stream's and its
 * helpers' queued work; a later call on the stream creates them again.  Not
 * to be called while another host thread issues work of this library on the
 * same stream.  A stream with no such state: nothing to do, 0.
 */
int ifk_release_stream_state(void* stream);

/*
 * Copy n int32 status words (device memory) into pinned host memory
 * (hipHostMalloc, or torch's pin_memory) by a kernel on the stream: the host
 * reads them once an event recorded behind this call has completed, with no
 * blocking read and no copy-engine transfer between the kernels around it.
 * No counterpart in the reference (its hooks read no device status,
 * activation_hooks.py:579-580, 642-643): it is for callers that decide a
 * status-dependent fallback later, such as the hooks' streaming folds in bf16
 * arithmetic.  n in [1, 2^20].
 */
int ifk_status_to_host(void* stream, const int32_t* status, int32_t* host_status, int64_t n);

/*
 * Streaming TSQR fold -- replaces streaming_tsqr_update(running_R, new_chunk)
 * (ifkfac/triangular.py:246-307) as called from the hooks
 * (ifkfac/activation_hooks.py:579, :642).
 *
 * R is an n x n fp32 buffer (ldr >= n) whose first r_in rows hold the running
 * factor (upper trapezoidal, r_in = 0 for "no data yet"); rows [r_in, n) are
 * overwritten.  X is the p x n chunk (dtype x_dtype, ldx >= n).  On return
 * rows [0, *r_out) of R hold the factor of [R_old; X] with a positive
 * diagonal, *r_out = min(r_in + p, n) -- the shape torch.linalg.qr(mode=
 * "reduced") gives the reference -- and the remaining rows are zero.
 * X is not modified.
 */
size_t ifk_tsqr_fold_workspace_size(int64_t p, int64_t n);
int ifk_tsqr_fold(void* stream, const void* X, int x_dtype, int64_t p, int64_t n, int64_t ldx,
                  float* R, int64_t ldr, int64_t r_in, int math, void* workspace,
                  size_t workspace_bytes, int64_t* r_out);

/*
 * Damped finalisation -- replaces the `R_raw / sqrt(rows)` scaling and
 * finalize_R(R, damping) of get_factors (ifkfac/activation_hooks.py:328-332,
 * ifkfac/triangular.py:386-421) and, with out_dtype = IFK_BF16, the RNE cast
 * of _update_factors (ifkfac/ifkfac.py:292-294).
 *
 * out (n x n, ldo) = R_d with R_d^T R_d = scale^2 R_in^T R_in + damping I,
 * upper triangular with positive diagonal.  If `finite` is non-null, *finite
 * is set to 1 if every entry of R_d is finite and 0 otherwise (the check of
 * ifkfac/ifkfac.py:232), written on the stream.
 */
size_t ifk_finalize_workspace_size(int64_t n);
int ifk_finalize(void* stream, const float* R_in, int64_t ldr_in, int64_t n, float scale,
                 float damping, void* out, int out_dtype, int64_t ldo, int math, int32_t* finite,
                 void* workspace, size_t workspace_bytes);

/*
 * Fold and finalize in one factorisation -- replaces the last
 * streaming_tsqr_update of a factor window (ifkfac/triangular.py:246-307)
 * followed by get_factors' scaling and finalize_R (ifkfac/activation_hooks.py:
 * 328-332, ifkfac/triangular.py:386-421) when the undamped running factor is
 * discarded right after, as IFKFAC._update_factors does (get_factors, then
 * hooks.clear(): ifkfac/ifkfac.py:208, 227).
 *
 * out (n x n, ldo) = R_d with
 *   R_d^T R_d = scale^2 (R_in^T R_in + X^T X) + damping I,
 * upper triangular with positive diagonal, where R_in holds the r_in rows
 * folded so far (row-major, ldr; entries below its diagonal are ignored) and
 * X (p x n, ldx, fp32 or bf16) is the last chunk.  The result is the R of
 * [scale R_in; scale X; sqrt(damping) I], computed as one TPQRT fold of
 * [R_in; X] under the triangular block sqrt(damping) / scale I.  `finite` as
 * for ifk_finalize.  Neither R_in nor X is modified.  With damping == 0,
 * r_in + p must be at least n.
 */
size_t ifk_fold_finalize_workspace_size(int64_t p, int64_t n, int64_t r_in);
int ifk_fold_finalize(void* stream, const void* X, int x_dtype, int64_t p, int64_t n,
                      int64_t ldx, const float* R_in, int64_t ldr, int64_t r_in, float scale,
                      float damping, void* out, int out_dtype, int64_t ldo, int math,
                      int32_t* finite, void* workspace, size_t workspace_bytes);

/*
 * ifk_fold_finalize with each 1024-column outer block of the TPQRT fold
 * factored at once by CholeskyQR2 with Householder reconstruction, instead
 * of by its chain of 64-column panels: the block's work becomes a few large
 * MFMA products and 1024 x 1024 factorisations.  No counterpart in the
 * reference (its fold is torch.linalg.qr, ifkfac/triangular.py:284-301 and
 * :411-416); same arguments and result as ifk_fold_finalize, for callers
 * that can read a status flag before using the factor.  *status (device):
 *   1  the factor is finite;
 *   0  it is not (non-finite input);
 *   2  some block was too ill-conditioned for CholeskyQR (a Cholesky pivot
 *      below 1e-4 of its diagonal in the first pass, or below 1/4 in the
 *      second): the output is meaningless and ifk_fold_finalize, on the same
 *      inputs, computes the factor.
 * status must not be NULL.
 */
size_t ifk_fold_finalize_cqr_workspace_size(int64_t p, int64_t n, int64_t r_in);
int ifk_fold_finalize_cqr(void* stream, const void* X, int x_dtype, int64_t p, int64_t n,
                          int64_t ldx, const float* R_in, int64_t ldr, int64_t r_in, float scale,
                          float damping, void* out, int out_dtype, int64_t ldo, int math,
                          int32_t* status, void* workspace, size_t workspace_bytes);

/*
 * ifk_fold_finalize from the Gram matrix instead of a TPQRT fold, in bf16
 * arithmetic (math must be IFK_MATH_BF16): A = P^T P + (damping / scale^2) I
 * with P = [R_in; X] rounded to bf16 (exact products, fp32 accumulation), the
 * factor R = scale * chol(A) by a right-looking Cholesky over 1024-column
 * blocks whose panel and Schur-update products keep fp32 accuracy by
 * splitting each operand into two bf16 halves.  No counterpart in the
 * reference (its fold is torch.linalg.qr, ifkfac/triangular.py:284-301 and
 * :411-416, whose R is the same unique factor); same arguments and result as
 * ifk_fold_finalize_cqr.  *status (device): 1 finite, 0 not finite, 2 some
 * pivot fell below 1e-3 of its column's Gram diagonal (more cancellation
 * than the Gram matrix's rounding leaves room for): the output is then
 * meaningless and ifk_fold_finalize, on the same inputs, computes the
 * factor.  status must not be NULL.  kappa_bound (device float, may be
 * NULL) receives an upper bound of kappa_2(R) from the Gram matrix,
 * sqrt(1 + ||scale^2 P^T P||_F / damping) (infinite without damping): the
 * choice between bf16 and fp32-accurate solves needs no power iteration.
 */
size_t ifk_fold_finalize_gram_workspace_size(int64_t p, int64_t n, int64_t r_in);
int ifk_fold_finalize_gram(void* stream, const void* X, int x_dtype, int64_t p, int64_t n,
                           int64_t ldx, const float* R_in, int64_t ldr, int64_t r_in, float scale,
                           float damping, void* out, int out_dtype, int64_t ldo, int math,
                           int32_t* status, float* kappa_bound, void* workspace,
                           size_t workspace_bytes);

/*
 * The streaming fold by the Gram route -- replaces streaming_tsqr_update
 * (ifkfac/triangular.py:246-307) in bf16 arithmetic when the folded factor is
 * square (r_in + p >= n): R (n x n fp32, rows [0, r_in) valid) becomes the
 * upper factor with positive diagonal of [R[0:r_in]; X] from its Gram matrix
 * and the blocked Cholesky of ifk_fold_finalize_gram.  The chunk enters as its
 * RNE bf16 rounding; the running factor, fp32 state that every fold of a
 * stream reads again, enters split as hi + lo (two bf16 halves: R^T R to
 * about 2^-17, three products over its rows) -- rounded to bf16 at every
 * fold, it would drift (0.28 relative Gram error after 200 folds of 4096 x
 * 768 chunks, against 2.5e-4 split).
 * *status: 1 R written; 2 a pivot fell below pivot_tol times its Gram
 * diagonal (too ill-conditioned for the Gram route at that tolerance) or the
 * input is not finite.  R is left unchanged unless *status is 1, so the caller
 * folds by ifk_tsqr_fold instead (the host reads the status).  pivot_tol in
 * (0, 1).
 */
size_t ifk_tsqr_fold_gram_workspace_size(int64_t p, int64_t n, int64_t r_in);
int ifk_tsqr_fold_gram(void* stream, const void* X, int x_dtype, int64_t p, int64_t n,
                       int64_t ldx, float* R, int64_t ldr, int64_t r_in, float pivot_tol,
                       int32_t* status, void* workspace, size_t workspace_bytes);

/*
 * ifk_tsqr_fold_gram for `batch` running factors of one shape, each folding
 * its own chunk (X[e], p x n), in one chain of launches -- replaces the
 * per-layer folds of the bucketed flush (ifkfac/activation_hooks.py:370-457,
 * its batched_qr over same-shape layers, triangular.py:331-379).  R[e]
 * (n x n fp32, ldr, rows [0, r_in) valid) and status[e] (device) are exactly
 * what ifk_tsqr_fold_gram gives that entry alone: 1 and R[e] the factor of
 * [R[e][0:r_in]; X[e]], or 2 and R[e] untouched (the caller folds that entry
 * by ifk_tsqr_fold).  X and R are host arrays of device pointers.
 */
size_t ifk_tsqr_fold_gram_batched_workspace_size(int64_t batch, int64_t p, int64_t n,
                                                 int64_t r_in);
int ifk_tsqr_fold_gram_batched(void* stream, int64_t batch, const void* const* X, int x_dtype,
                               int64_t p, int64_t n, int64_t ldx, float* const* R, int64_t ldr,
                               int64_t r_in, float pivot_tol, int32_t* status, void* workspace,
                               size_t workspace_bytes);

/*
 * ifk_fold_finalize_gram for `batch` layers of the same shape in the same
 * launches (replaces the per-layer loop of batched_streaming_tsqr_update /
 * flush, ifkfac/triangular.py:331-379, ifkfac/activation_hooks.py:370-457,
 * for the factor update of a bucket of same-shape layers): every launch of
 * the latency-bound Cholesky chain serves all of them.  X and R_in are HOST
 * arrays of `batch` device pointers (R_in may be NULL when r_in == 0); entry
 * b's factor is written at out + b * out_stride elements (out_stride >= n *
 * ldo), its status to status[b] and its kappa bound to kappa_bound[b] (may be
 * NULL).  pivot_tol in (0, 1) is the relative pivot threshold of the
 * status (ifk_fold_finalize_gram uses 1e-3).  Every entry's result is the one
 * ifk_fold_finalize_gram gives it at that threshold.
 */
size_t ifk_fold_finalize_gram_batched_workspace_size(int64_t batch, int64_t p, int64_t n,
                                                     int64_t r_in);
int ifk_fold_finalize_gram_batched(void* stream, int64_t batch, const void* const* X, int x_dtype,
                                   int64_t p, int64_t n, int64_t ldx, const float* const* R_in,
                                   int64_t ldr, int64_t r_in, float scale, float damping,
                                   void* out, int out_dtype, int64_t ldo, int64_t out_stride,
                                   int math, float pivot_tol, int32_t* status, float* kappa_bound,
                                   void* workspace, size_t workspace_bytes);

/*
 * ifk_fold_finalize_gram_batched together with the triangular inverse of each
 * factor and its bf16 copies (replaces finalize_R, ifkfac/triangular.py:
 * 386-421, and the solves of apply_vered on bf16 factors, triangular.py:
 * 608-628, whose inverse ifk_tri_inverse_bf16 would otherwise form after the
 * factor): Z = R^{-1} (fp32, upper, zero below), Zb = bf16(Z) (upper, zero
 * below) and ZTb = bf16(Z^T) (lower, zero above), the copies
 * ifk_precondition_apply_bf16 reads.  Z's diagonal 1024-blocks are the
 * inverses of the fp32 factor's diagonal blocks, which the blocked Cholesky
 * forms anyway; the rest comes from the block-doubling levels of
 * ifk_tri_inverse_bf16 on `out` (bf16 arithmetic, fp32 accumulation), which
 * start at width 1024 instead of at its 64-column leaves.  Entry b's Z at Z + b * z_stride
 * (ld ldz), its copies at Zb / ZTb + b * b_stride (ld ldb, bf16 elements).
 * The factor, status and kappa bound are bit for bit those of
 * ifk_fold_finalize_gram_batched; where an entry's status is 2 its inverse
 * is meaningless (the caller refactors that side and inverts it by
 * ifk_tri_inverse_bf16).  bf16 arithmetic only (no math argument).
 */
size_t ifk_fold_finalize_gram_inverse_workspace_size(int64_t batch, int64_t p, int64_t n,
                                                     int64_t r_in);
int ifk_fold_finalize_gram_inverse(void* stream, int64_t batch, const void* const* X, int x_dtype,
                                   int64_t p, int64_t n, int64_t ldx, const float* const* R_in,
                                   int64_t ldr, int64_t r_in, float scale, float damping,
                                   void* out, int out_dtype, int64_t ldo, int64_t out_stride,
                                   float pivot_tol, int32_t* status, float* kappa_bound, float* Z,
                                   int64_t ldz, int64_t z_stride, void* Zb, void* ZTb, int64_t ldb,
                                   int64_t b_stride, void* workspace, size_t workspace_bytes);

/*
 * Triangular inverse Z = R^{-1} of an upper-triangular n x n factor (dtype
 * r_dtype) into fp32 Z (ldz).  The four solves of apply_vered are applied as
 * products with Z; this is the factor-side half of them.
 */
size_t ifk_tri_inverse_workspace_size(int64_t n);
int ifk_tri_inverse(void* stream, const void* R, int r_dtype, int64_t ldr, int64_t n, float* Z,
                    int64_t ldz, int math, void* workspace, size_t workspace_bytes);

/*
 * ifk_tri_inverse in bf16 arithmetic that also hands back RNE bf16 copies
 * Zb = Z and ZTb = Z^T (row stride ldb, the other triangle zero), the
 * operands ifk_precondition_apply_bf16 reads without casting them again.
 * No counterpart in the reference (its solves run per step on R); for
 * callers that keep the inverses between factor updates.
 */
size_t ifk_tri_inverse_bf16_workspace_size(int64_t n);
int ifk_tri_inverse_bf16(void* stream, const void* R, int r_dtype, int64_t ldr, int64_t n,
                         float* Z, int64_t ldz, void* Zb, void* ZTb, int64_t ldb, void* workspace,
                         size_t workspace_bytes);

/*
 * ifk_tri_inverse at about fp32 accuracy on bf16 MFMA: the wide doubling
 * levels multiply split bf16 halves (x = x_hi + x_lo; three products per
 * product, about 2^-17 of |a||b| each, two when R is bf16-valued), the
 * 128-blocks and the levels up to 256 wide run in fp32 arithmetic.  The
 * fp32 solves on bf16-valued factors of triangular.py:607-628 use this
 * inverse with ifk_precondition_apply_x3 (same accuracy class); about 4x
 * faster than ifk_tri_inverse in fp32 arithmetic at n = 4096.  Workspace
 * about 8 n^2 bytes plus 4 n^2 more for an fp32 R.
 */
size_t ifk_tri_inverse_x3_workspace_size(int64_t n, int r_dtype);
int ifk_tri_inverse_x3(void* stream, const void* R, int r_dtype, int64_t ldr, int64_t n, float* Z,
                       int64_t ldz, void* workspace, size_t workspace_bytes);

/*
 * Condition estimate kappa_2(R) ~ sigma_max(R) sigma_max(Z) of an upper-
 * triangular n x n factor R (dtype r_dtype, ldr) from R and its inverse Z
 * (fp32, ldz, e.g. from ifk_tri_inverse_bf16), each sigma_max by four steps
 * of block power iteration with four deterministic probe vectors; the result
 * (a lower bound, within a few percent when the extreme singular values are
 * spread, about 10 % when they cluster) is written on the stream to the
 * device float *kappa.  No
 * counterpart in the reference; IFKFAC uses it to choose the arithmetic of a
 * layer's solves in bf16 mode (bf16 where the factors are near-isotropic,
 * fp32 as the reference's triangular.py:621-628 otherwise).
 */
size_t ifk_cond_estimate_workspace_size(int64_t n);
int ifk_cond_estimate(void* stream, const void* R, int r_dtype, int64_t ldr, const float* Z,
                      int64_t ldz, int64_t n, float* kappa, void* workspace,
                      size_t workspace_bytes);

/*
 * Four triangular solves -- replaces apply_vered(grad_W, R_X, R_G)
 * (ifkfac/triangular.py:551-656) and the per-entry body of
 * apply_vered_batched (ifkfac/triangular.py:430-451, :506-544):
 *   nat = (R_G^T R_G)^{-1} grad (R_X^T R_X)^{-1}
 * grad and nat are n_out x n_in fp32.  ifk_precondition takes the factors;
 * ifk_precondition_apply takes their inverses from ifk_tri_inverse, which
 * lets a caller reuse them for every step between factor updates.
 */
size_t ifk_precondition_workspace_size(int64_t n_out, int64_t n_in, int math);
int ifk_precondition(void* stream, const float* grad, int64_t n_out, int64_t n_in, int64_t ldg,
                     const void* R_X, int64_t ldrx, const void* R_G, int64_t ldrg, int r_dtype,
                     float* nat, int64_t ldn, int math, void* workspace, size_t workspace_bytes);

size_t ifk_precondition_apply_workspace_size(int64_t n_out, int64_t n_in, int math);
int ifk_precondition_apply(void* stream, const float* grad, int64_t n_out, int64_t n_in,
                           int64_t ldg, const float* Z_X, int64_t ldzx, const float* Z_G,
                           int64_t ldzg, float* nat, int64_t ldn, int math, void* workspace,
                           size_t workspace_bytes);
/* the same in bf16 arithmetic from the copies of ifk_tri_inverse_bf16 */
size_t ifk_precondition_apply_bf16_workspace_size(int64_t n_out, int64_t n_in);
int ifk_precondition_apply_bf16(void* stream, const float* grad, int64_t n_out, int64_t n_in,
                                int64_t ldg, const void* Z_Xb, const void* Z_Xt, int64_t ldzx,
                                const void* Z_Gb, const void* Z_Gt, int64_t ldzg, float* nat,
                                int64_t ldn, void* workspace, size_t workspace_bytes);

/*
 * The apply at fp32 accuracy on bf16 MFMA, for factors whose kappa_2 makes the
 * bf16 apply's rounding visible (IFKFAC's bf16 mode takes it when the factor
 * update's kappa bound exceeds 1.5; the reference's bf16 mode solves in fp32
 * on the bf16-valued factors, ifkfac/triangular.py:621-628).  Every product of
 * nat = Z_G Z_G^T grad Z_X Z_X^T is formed from bf16 halves x = x_hi + x_lo as
 * a_hi b_hi + a_hi b_lo + a_lo b_hi (three MFMA launches into one fp32 result,
 * about 2^-17 of |a||b| per product).  ifk_inverse_split_copies makes a side's
 * halves from its fp32 inverse Z (tri_inverse): Z_hi, Z_lo (row-major) and
 * ZT_hi, ZT_lo (Z^T), all n x n bf16 with row stride ldb.
 */
int ifk_inverse_split_copies(void* stream, const float* Z, int64_t ldz, int64_t n, void* Z_hi,
                             void* Z_lo, void* ZT_hi, void* ZT_lo, int64_t ldb);
size_t ifk_precondition_apply_x3_workspace_size(int64_t n_out, int64_t n_in);
int ifk_precondition_apply_x3(void* stream, const float* grad, int64_t n_out, int64_t n_in,
                              int64_t ldg, const void* Z_X_hi, const void* Z_X_lo,
                              const void* Z_XT_hi, const void* Z_XT_lo, int64_t ldzx,
                              const void* Z_G_hi, const void* Z_G_lo, const void* Z_GT_hi,
                              const void* Z_GT_lo, int64_t ldzg, float* nat, int64_t ldn,
                              void* workspace, size_t workspace_bytes);

/*
 * ifk_precondition_apply_bf16 without a workspace argument: its scratch is a
 * 64 MiB device array inside this library (one per GPU, held until the
 * process ends), so the call allocates nothing.  No counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and result as ifk_precondition_apply_bf16, bit for bit while the
 * array also has room for that entry's split-K scratch.  Limit: the three bf16
 * n_out x n_in intermediates must fit in the array (n_out * n_in up to about
 * 11.18 million; larger calls return IFK_ERR_INVALID).  The stream's device
 * must be the current device.  All calls on one GPU share the array: calls
 * that overlap on one GPU (other streams, other threads) race.
 */
int ifk_precondition_apply_bf16_noalloc(void* stream, const float* grad, int64_t n_out,
                                        int64_t n_in, int64_t ldg, const void* Z_Xb,
                                        const void* Z_Xt, int64_t ldzx, const void* Z_Gb,
                                        const void* Z_Gt, int64_t ldzg, float* nat, int64_t ldn);

/*
 * Bias preconditioning -- replaces apply_vered_bias(grad_b, R_G)
 * (ifkfac/triangular.py:659-705): out = (R_G^T R_G)^{-1} g, given Z_G.
 */
/*
 * The two per-step applies for `batch` layers of one shape in grouped
 * launches -- replaces apply_vered_batched (ifkfac/triangular.py:506-544, the
 * bucketed apply of ifkfac/ifkfac.py:371-380): each of the four products (in
 * the _x3 form each split product) is one launch over the batch, and every
 * entry's nat is bit for bit what ifk_precondition_apply_bf16 /
 * ifk_precondition_apply_x3 give that layer alone.  grad is a host array of
 * `batch` device pointers (n_out x n_in fp32, ldg each); the inverse copies
 * (and their halves) of entry e sit at e * stride_zx / e * stride_zg elements
 * from the given ones, and nat of entry e at e * stride_nat.
 */
size_t ifk_precondition_apply_bf16_batched_workspace_size(int64_t batch, int64_t n_out,
                                                         int64_t n_in);
int ifk_precondition_apply_bf16_batched(void* stream, int64_t batch, const float* const* grad,
                                        int64_t n_out, int64_t n_in, int64_t ldg,
                                        const void* Z_Xb, const void* Z_Xt, int64_t ldzx,
                                        int64_t stride_zx, const void* Z_Gb, const void* Z_Gt,
                                        int64_t ldzg, int64_t stride_zg, float* nat, int64_t ldn,
                                        int64_t stride_nat, void* workspace,
                                        size_t workspace_bytes);
size_t ifk_precondition_apply_x3_batched_workspace_size(int64_t batch, int64_t n_out,
                                                       int64_t n_in);
int ifk_precondition_apply_x3_batched(void* stream, int64_t batch, const float* const* grad,
                                      int64_t n_out, int64_t n_in, int64_t ldg,
                                      const void* Z_X_hi, const void* Z_X_lo, const void* Z_XT_hi,
                                      const void* Z_XT_lo, int64_t ldzx, int64_t stride_zx,
                                      const void* Z_G_hi, const void* Z_G_lo, const void* Z_GT_hi,
                                      const void* Z_GT_lo, int64_t ldzg, int64_t stride_zg,
                                      float* nat, int64_t ldn, int64_t stride_nat,
                                      void* workspace, size_t workspace_bytes);

size_t ifk_precondition_bias_workspace_size(int64_t n_out);
int ifk_precondition_bias(void* stream, const float* g, int64_t n_out, const float* Z_G,
                          int64_t ldzg, float* out, void* workspace, size_t workspace_bytes);

/*
 * Momentum and weight update -- replaces the per-layer update of
 * _apply_preconditioner_bucketed (ifkfac/ifkfac.py:402-413) and
 * _apply_preconditioner (ifkfac/ifkfac.py:500-510) as one pass:
 *   buf = buf_init ? nat : momentum * buf + nat      (momentum > 0 only)
 *   W   = W * (1 - lr * weight_decay) - lr * (momentum > 0 ? buf : nat)
 * (the decay factor only when weight_decay > 0).  All arrays fp32, numel
 * elements; buf may be null when momentum == 0.
 */
int ifk_momentum_update(void* stream, const float* nat, float* buf, float* W, int64_t numel,
                        float lr, float momentum, float weight_decay, int buf_init);

/*
 * R factor of a tall matrix -- replaces block_householder_qr_bf16 and
 * householder_qr_bf16 (ifkfac/bf16_linalg.py:64-153, :158-183).
 * A is m x n (m >= n); R (n x n, r_dtype) is upper triangular with a positive
 * diagonal.
 */
size_t ifk_geqrf_r_workspace_size(int64_t m, int64_t n);
int ifk_geqrf_r(void* stream, const void* A, int a_dtype, int64_t m, int64_t n, int64_t lda,
                void* R, int r_dtype, int64_t ldr, int math, void* workspace,
                size_t workspace_bytes);

/*
 * Triangular solve -- replaces solve_triangular_bf16(R, B, upper)
 * (ifkfac/bf16_linalg.py:188-242): X = R^{-1} B (upper != 0) or L^{-1} B,
 * R n x n, B and X n x k.  Diagonal divisors follow _safe_div
 * (ifkfac/bf16_linalg.py:44-59).
 */
size_t ifk_trsm_workspace_size(int64_t n, int64_t k);
int ifk_trsm(void* stream, const void* R, int r_dtype, int64_t n, int64_t ldr, int upper,
             const void* B, int b_dtype, int64_t k, int64_t ldb, void* X, int x_dtype, int64_t ldx,
             int math, void* workspace, size_t workspace_bytes);

/*
 * Cholesky -- replaces cholesky_bf16(A) (ifkfac/bf16_linalg.py:247-267):
 * L lower with L L^T = A, pivots clamped at 1e-7 as the reference does.
 */
size_t ifk_potrf_workspace_size(int64_t n);
int ifk_potrf(void* stream, const void* A, int a_dtype, int64_t n, int64_t lda, void* L,
              int l_dtype, int64_t ldl, int math, void* workspace, size_t workspace_bytes);

/*
 * SPD inverse -- replaces inv_spd_bf16(A) (ifkfac/bf16_linalg.py:272-280).
 */
size_t ifk_inv_spd_workspace_size(int64_t n);
int ifk_inv_spd(void* stream, const void* A, int a_dtype, int64_t n, int64_t lda, void* X,
                int x_dtype, int64_t ldx, int math, void* workspace, size_t workspace_bytes);

/*
 * Classic K-FAC control (the reference's explicit-Gram baseline, kept to
 * contrast the kappa^2 of forming X^T X with the factor path's kappa):
 *   ifk_gram_accumulate   S = beta S + X^T X, full symmetric fp32 n x n, in the
 *                         arithmetic of the activations' dtype -- replaces
 *                         `x.t().mm(x)` + `A_sum.add_` of KFACHooks' hooks
 *                         (ifkfac/kfac_hooks.py:208-214, :239-245);
 *   ifk_inv_spd_damped    X = (A + damping I)^{-1} in fp32 by Cholesky (pivots
 *                         clamped at 1e-7) and the triangular inverse --
 *                         replaces `A + damping * eye` + `torch.linalg.inv`
 *                         (ifkfac/classic_kfac.py:131-138);
 *   ifk_classic_precondition  nat = G_inv grad A_inv in fp32 -- replaces
 *                         `G_inv @ grad_w @ A_inv` (ifkfac/classic_kfac.py:218).
 */
size_t ifk_gram_accumulate_workspace_size(int64_t n);
int ifk_gram_accumulate(void* stream, const void* X, int x_dtype, int64_t p, int64_t n,
                        int64_t ldx, float* S, int64_t lds, float beta, void* workspace,
                        size_t workspace_bytes);
/* Y = alpha X + beta Y (fp32 rows x cols; beta == 0 does not read Y): the
 * Gram averages A_sum / n_A (kfac_hooks.py:263-264) and the EMA blend
 * gamma A_old + (1 - gamma) A_new (classic_kfac.py:113-120). */
int ifk_axpby(void* stream, float alpha, const float* X, int64_t ldx, float beta, float* Y,
              int64_t ldy, int64_t rows, int64_t cols);
size_t ifk_inv_spd_damped_workspace_size(int64_t n);
int ifk_inv_spd_damped(void* stream, const void* A, int a_dtype, int64_t n, int64_t lda,
                       float damping, float* X, int64_t ldx, void* workspace,
                       size_t workspace_bytes);
size_t ifk_classic_precondition_workspace_size(int64_t n_out, int64_t n_in);
int ifk_classic_precondition(void* stream, const float* grad, int64_t n_out, int64_t n_in,
                             int64_t ldg, const float* A_inv, int64_t ldai, const float* G_inv,
                             int64_t ldgi, float* nat, int64_t ldn, void* workspace,
                             size_t workspace_bytes);

/*
 * Laplace consumer of the factors (the K-FAC Laplace posterior of
 * ifkfac/laplace.py, fed by hooks.get_factors() as README.md:146-171 shows):
 *   ifk_factor_evd      R^T R = V diag(eigvals) V^T from the n x n factor R (its
 *                       upper triangle), by one-sided block Jacobi SVD of R:
 *                       V (n x n fp32, columns = right singular vectors of R),
 *                       eigvals = sigma(R)^2 descending; *sweeps = Jacobi sweeps
 *                       to convergence (negative: not converged).  This is the
 *                       `factors_to_evd` the reference's README names
 *                       (README.md:167) and never defines: svd(R) per factor
 *                       (laplace.py:26-30);
 *   ifk_laplace_scales  out = 1 / sqrt(sqrt_n d + sqrt_lam) -- replaces
 *                       laplace.py:95-96;
 *   ifk_laplace_sample  W = W_map + U_G diag(s_G) Xi diag(s_A) U_A^T (fp32) --
 *                       replaces laplace.py:138-154 (Xi drawn by the caller).
 */
size_t ifk_factor_evd_workspace_size(int64_t n);
int ifk_factor_evd(void* stream, const void* R, int r_dtype, int64_t ldr, int64_t n, float* V,
                   int64_t ldv, float* eigvals, int* sweeps, void* workspace,
                   size_t workspace_bytes);
int ifk_laplace_scales(void* stream, const float* d, int64_t n, float sqrt_n, float sqrt_lam,
                       float* out);
size_t ifk_laplace_sample_workspace_size(int64_t n_out, int64_t n_in);
int ifk_laplace_sample(void* stream, const float* W_map, int64_t ldm, float* W, int64_t ldw,
                       int64_t n_out, int64_t n_in, const float* U_G, int64_t ldug,
                       const float* s_G, const float* U_A, int64_t ldua, const float* s_A,
                       const float* Xi, int64_t ldxi, void* workspace, size_t workspace_bytes);

/*
 * General MFMA matrix product C = alpha op(A) op(B) + beta C, exposed for
 * tests and for callers that compose the path themselves.  Bit 0 of
 * trans_a/trans_b selects op(X) = X^T; bits 1-2 declare op(X) upper (1) or
 * lower (2) triangular, whose other triangle is then never read.  C is fp32.
 */
size_t ifk_gemm_workspace_size(int64_t m, int64_t n);
int ifk_gemm(void* stream, int math, int64_t m, int64_t n, int64_t k, float alpha, const void* A,
             int a_dtype, int64_t lda, int trans_a, const void* B, int b_dtype, int64_t ldb,
             int trans_b, float beta, float* C, int64_t ldc, void* workspace,
             size_t workspace_bytes);

/*
 * Measurement support (no counterpart in the reference; used by bench.py).
 * ifk_profile_begin(v) arms the GEMM launch profiler for GEMM variant v
 * (v = (streamk << 9) | (mid << 7) | (direct << 6) | (large_tile << 5) |
 * (math << 4) | (a_dtype << 3) | (a_k_contiguous << 2) | (b_dtype << 1) |
 * b_k_contiguous; large_tile marks the bf16 kernels with the large tiles,
 * direct the one that loads operands straight into LDS, gemm_bb_kernel, mid
 * its 128 x 128 tile and streamk a launch of it that walks the tiles
 * stream-K; large_tile alone gemm_big_kernel, neither gemm_kernel; the
 * block Cholesky's launches have v = 4096 (cholb_first_kernel) and 4097
 * (cholb_step_kernel)), for every variant with v = -2, for every launch of
 * gemm_big_kernel with v = -3, of gemm_kernel with v = -4, of gemm_bb_kernel
 * with its 256 x 256 tile with v = -5 and with its 128 x 128 tile with v = -6,
 * of cholb_first_kernel with v = -7 and of cholb_step_kernel with v = -8;
 * v = -1 disarms.  A block-Cholesky launch's algorithmic flops are its even
 * share of n^3 / 3 for the factor plus n^3 / 3 for its inverse.
 * Each armed launch is bracketed by two HIP events on its own stream.
 * ifk_profile_end() disarms, waits for the events and returns the number of
 * launches recorded; ifk_profile_get(i, ...) returns launch i's variant,
 * duration (ms), algorithmic flops and bytes, and its m, n, k.
 */
int ifk_profile_begin(int variant);
int ifk_profile_end(int64_t* n_launches);

int ifk_profile_get(int64_t i, int* variant, float* ms, double* flops, double* bytes, int64_t* m,
                    int64_t* n, int64_t* k);

#ifdef __cplusplus
}
#endif

#endif /* IFKFAC_HIP_H */
