// Host-side launchers of the single-purpose kernels (small.hip, panel.hip,
// elementwise.hip).
#pragma once
#include "common.h"

namespace ifk {

// --- panel step of the fold (small.hip, panel.hip); b <= 64 ------------------
// Gram matrices over row slabs: part[(s * ncb + cb) * 4096] (64 x 64 each)
// for gram_slabs(pe) 128-row slabs s and 64-column blocks cb (at most
// PANEL_MAX_CB), reduced in slab order into G[cb * 4096].
constexpr int PANEL_MAX_CB = 8;
int gram_slabs(int64_t pe);
// G = A^T [B0 | B1] over the pe rows: A (at most 64 wide) stored transposed
// when a_ts (else row-major), B0 optional, row-major and at most 64 wide, B1
// (w1 wide) stored transposed; *ncb_out = number of 64-column blocks of G.
int launch_gram(hipStream_t s, const float* A, int64_t lda, int ka, bool a_ts, const float* B0,
                int64_t ldb0, int w0, const float* B1, int64_t ldb1, int w1, int64_t pe,
                float* part, float* G, int* ncb_out);
// CholeskyQR pass 1: G1 (+ P_top^T P_top) = U1^T U1, M1 = U1^{-1},
// Q1 = P_top M1; *flag = 1 when a pivot falls below tol * its diagonal.
int launch_panel_hr_a(hipStream_t s, const float* G, const float* Ptop, int64_t ldr, int b,
                      float tol, float* U1, float* M1, float* Q1, int* flag);
// Q2 = X_p M1 (X_p given transposed, XT b x pe); when *flag is set, the
// Householder TPQRT of [P_top; X_p] instead: reflectors into Q2 (ld 64,
// columns >= b zero), P_top <- R_new.
int launch_apply_m(hipStream_t s, const float* XT, int64_t ldx, int64_t pe, int b, const float* M,
                   float* Q2, float* Ptop, int64_t ldr, const int* flag);
// CholeskyQR pass 2 + Householder reconstruction from G2 (+ Q1^T Q1) (for a
// flagged panel T from the UT transform of Y^T Y, N = I, NT = T): N (ld b),
// R_new into R's diagonal block, and for each 64-column block of the nr
// columns right of it (G block 1 + cb = Q2^T C_rest):
// W = NT^T (Q2^T C) + T^T R_rest, R_rest -= W, NW = N W (ld ldnw).
int launch_panel_hrw(hipStream_t s, const float* G, int ncb, const float* Q1, const float* U1,
                     int b, float* N, float* R, int64_t ldr, int nr, float* NW, int64_t ldnw,
                     const int* flag);
// Y = Q2 N (ld ldy; also RNE bf16 into Yb, same ld, when Yb is given, and
// into YbT transposed, b rows of ld ldt >= pe, when YbT is given) and
// CT_rest -= (Q2 NW)^T on the transposed working matrix (nr rows of ld ldc)
int launch_panel_update(hipStream_t s, const float* Q2, int64_t pe, int b, const float* N,
                        float* Y, int64_t ldy, bf16_t* Yb, bf16_t* YbT, int64_t ldt,
                        const float* NW, int64_t ldnw, float* CT, int64_t ldc, int nr);
// R_blk (rows x cols, ldr) -= WT^T (WT cols x rows, ldw)
int launch_sub_transposed(hipStream_t s, float* R, int64_t ldr, const float* WT, int64_t ldw,
                          int64_t rows, int64_t cols);
// Tinv = striu(G) + diag(1 + diag G) / 2 (UT transform of a reflector Gram matrix)
int launch_ut_tinv(hipStream_t s, const float* G, int64_t ldg, int64_t n, float* Tinv,
                   int64_t ldt);
int launch_chol_block(hipStream_t s, float* A, int64_t ld, int b);
// Blocked upper Cholesky A = U^T U of an n x n fp32 matrix, n <= 1024 (one
// launch per 64-column step; A's blocks right of the diagonal are
// overwritten by the trailing updates).  U (ld ldu) receives the blocks on
// and above the diagonal, Zd (ceil(n / 64) x 4096 floats) the inverses of the
// diagonal 64-blocks, dref (n floats) diag(A).  A pivot below tol * diag(A)_i
// sets *flag.
// With M (ld ldm), M = U^{-1} as well (its blocks on and above the diagonal),
// formed column block by column block alongside the factorisation.  With
// dref_in, dref holds the reference diagonal on entry instead (e.g. a Gram
// matrix's diagonal before the updates that produced A).  batch independent
// factorisations of the same size run in the same launches, entry b at the
// given element strides from each pointer (flag: int strides).
struct CholbStrides {
  int64_t a = 0, u = 0, zd = 0, dref = 0, m = 0, flag = 0;
};
int launch_cholb(hipStream_t s, float* A, int64_t lda, int n, float* U, int64_t ldu, float* Zd,
                 float* dref, float tol, int* flag, float* M = nullptr, int64_t ldm = 0,
                 bool dref_in = false, int batch = 1, CholbStrides bs = CholbStrides());
// hi = RNE bf16(src), lo = RNE bf16(src - hi); transposed (hi[c][r]) with trans
int launch_split_bf16(hipStream_t s, const float* src, int64_t lds, int64_t rows, int64_t cols,
                      bf16_t* hi, bf16_t* lo, int64_t ldo, bool trans = false);
// *status = 2 if *flag != 0
int launch_status_merge(hipStream_t s, int* status, const int* flag);
// (and, when given, RNE bf16 copies of the blocks into Zb row-major and into
// ZTb transposed, both of row stride ldb)
int launch_trinv_diag(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, int nb,
                      float* Z, int64_t ldz, int safe, bf16_t* Zb = nullptr,
                      bf16_t* ZTb = nullptr, int64_t ldb = 0);
// Diagonal 128 x 128 blocks of R^{-1} (R upper triangular, or with ut the UT
// transform striu(G) + diag(1 + diag G) / 2 of a reflector Gram matrix G =
// Y^T Y, whose inverse is the T factor of the reflectors [I; Y]); the last
// block may be ragged
int launch_trinv_diag128(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z,
                         int64_t ldz, int safe, int ut);
// Small product with a fused epilogue (sqmm_kernel in small.hip):
//   out = epi(alpha op(A) op(B) + beta1 C1 + beta2 C2 + gamma I)
enum SqEpi { SQ_PLAIN = 0, SQ_UP = 1, SQ_TRIU = 2 };
struct SqmmArgs {
  int64_t M = 0, N = 0, K = 0;
  const float* A = nullptr;
  int64_t lda = 0;
  int ta = 0, tria = TRI_NONE;
  const float* B = nullptr;
  int64_t ldb = 0;
  int tb = 0, trib = TRI_NONE;
  float alpha = 1.0f;
  const float* C1 = nullptr;
  int64_t ld1 = 0;
  float beta1 = 0.0f;
  const float* C2 = nullptr;
  int64_t ld2 = 0;
  float beta2 = 0.0f;
  float gamma = 0.0f;
  int epi = SQ_PLAIN;
  float* out = nullptr;
  int64_t ldo = 0;
  bf16_t* outb = nullptr;
  int64_t ldob = 0;
  int outb_t = 0;
  const float* prev = nullptr;
  float tol = 0.0f;
  int* flag = nullptr;
  float* out2 = nullptr;      // also up(v) (ld ldo), with epi == SQ_TRIU
  int vec_a = 0, vec_b = 0;   // set by launch_sqmm
};
constexpr int SQ_BATCH = 8;
struct SqmmBatch {
  SqmmArgs a[SQ_BATCH];
};
// count independent products (of any shapes) in one launch
int launch_sqmm(hipStream_t s, const SqmmArgs* a, int count = 1);
// C_b = alpha A_b B_b, fp32 row-major, 64 x 64 tiles (small products)
int launch_gemm64(hipStream_t s, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
                  int64_t lda, int64_t bsa, int tria, const float* B, int64_t ldb, int64_t bsb,
                  int trib, float* C, int64_t ldc, int64_t bsc, int batch);

// --- elementwise kernels (elementwise.hip) -----------------------------------
// dst (rows x cols, ldd, fp32) = scale * src (dtype sdt, lds)
int launch_copy_to_f32(hipStream_t s, const void* src, int sdt, int64_t lds, int64_t rows,
                       int64_t cols, float scale, float* dst, int64_t ldd);
// dst = scale * src restricted to the upper triangle (strict lower part set 0)
int launch_copy_upper(hipStream_t s, const float* src, int64_t lds, int64_t n, float scale,
                      float* dst, int64_t ldd);
// dst (n x n) = diag(value)
int launch_set_diag(hipStream_t s, float* dst, int64_t ldd, int64_t n, float value);
// rows [r0, r1) of dst (cols wide) set to zero
int launch_zero_rows(hipStream_t s, float* dst, int64_t ldd, int64_t r0, int64_t r1, int64_t cols);
// zero a rows x cols block
int launch_zero(hipStream_t s, float* dst, int64_t ldd, int64_t rows, int64_t cols);
int launch_zero_bf16(hipStream_t s, bf16_t* dst, int64_t ldd, int64_t rows, int64_t cols);
// zero the 64 x 64 blocks of an n x n matrix (element size es, ld elements)
// strictly below (lower) or above the block diagonal
int launch_zero_tri_blocks(hipStream_t s, void* dst, int es, int64_t ld, int64_t n, bool lower);
// dst -= src (rows x cols)
int launch_sub_inplace(hipStream_t s, float* dst, int64_t ldd, const float* src, int64_t lds,
                       int64_t rows, int64_t cols);
// negate rows i < r whose diagonal entry is negative (sign(0) counts as +)
int launch_sign_normalize(hipStream_t s, float* R, int64_t ldr, int64_t r, int64_t n);
// out (dtype odt) = R upper triangle (RNE for bf16); *finite &= all finite
int launch_cast_upper(hipStream_t s, const float* R, int64_t ldr, int64_t n, void* out, int odt,
                      int64_t ldo, int* finite, float scale = 1.0f);
// out (odt) = src (fp32), full matrix
int launch_cast(hipStream_t s, const float* src, int64_t lds, int64_t rows, int64_t cols, void* out,
                int odt, int64_t ldo);
// *flag = 1 (a one-thread fill, safe to capture in a graph)
int launch_fill_int(hipStream_t s, int* p, int value, int count);
// n status words from device memory to pinned host memory, by a kernel
// (dst_dev: the host buffer's device address)
int launch_status_to_host(hipStream_t s, const int* src, int* dst_dev, int n);
// heavy-ball momentum + decoupled weight decay + SGD step
int launch_momentum_update(hipStream_t s, const float* nat, float* buf, float* W, int64_t numel,
                           float lr, float momentum, float weight_decay, int buf_init);
// dst (cols x rows, fp32) = src^T (src rows x cols, dtype sdt); with upper set,
// entries of src below its diagonal are taken as zero
int launch_transpose_to_f32(hipStream_t s, const void* src, int sdt, int64_t lds, int64_t rows,
                            int64_t cols, float* dst, int64_t ldd, bool upper = false);
// out (odt, n x n) = lower triangle of src^T, i.e. out[i][j] = src[j][i] for j <= i, else 0
int launch_transpose_upper(hipStream_t s, const float* src, int64_t lds, int64_t n, void* out,
                           int odt, int64_t ldo);
// out[c][r] (odt) = src[r][c] for a rows x cols fp32 block; batched with
// element strides bss (src) and bso (out)
int launch_transpose_cast(hipStream_t s, const float* src, int64_t lds, int64_t rows, int64_t cols,
                          void* out, int odt, int64_t ldo, int batch = 1, int64_t bss = 0,
                          int64_t bso = 0);
// hi, lo (cols x rows, ldo) = the bf16 halves of src^T (src rows x cols fp32):
// hi = RNE(x), lo = RNE(x - hi)
int launch_split_transpose(hipStream_t s, const float* src, int64_t lds, int64_t rows,
                           int64_t cols, bf16_t* hi, bf16_t* lo, int64_t ldo);
// dst[c][r] = src[r][c] for a rows x cols bf16 block
int launch_transpose_bf16(hipStream_t s, const bf16_t* src, int64_t lds, int64_t rows,
                          int64_t cols, bf16_t* dst, int64_t ldd);
// A[i][i] += v, i < n
int launch_add_diag(hipStream_t s, float* A, int64_t lda, int64_t n, float v);
// Y = alpha X + beta Y (fp32); beta == 0 does not read Y
int launch_axpby(hipStream_t s, float alpha, const float* X, int64_t ldx, float beta, float* Y,
                 int64_t ldy, int64_t rows, int64_t cols);
// S[c][r] = S[r][c] for r > c: a symmetric matrix from its lower triangle
int launch_mirror_lower(hipStream_t s, float* S, int64_t ld, int64_t n);
// condition-estimate helpers (elementwise.hip)
int launch_probe_init(hipStream_t s, float* V, int64_t n, int k);
int launch_colnorm(hipStream_t s, float* V, int64_t n, int k, float* ss);
int launch_cond_final(hipStream_t s, const float* ssa, const float* ssb, int k, float* kappa);
// out (dt) = alpha * x (fp32) with optional bf16 output
int launch_scale_copy_vec(hipStream_t s, const float* x, int64_t n, float alpha, void* out, int odt);

}  // namespace ifk
