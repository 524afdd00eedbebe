// Host orchestration of the curvature path (see linalg.h).
//
// Streaming fold (triangular.py:246-307, streaming_tsqr_update):
//   R (n x n, rows >= r_in zero) and a chunk X (p x n) are combined into the
//   R factor of [R; X] without forming Q, as a blocked triangular-pentagonal
//   Householder QR: for each 64-column panel the reflectors touch only the
//   panel's b rows of R and the rows of X, V = [I; Y].  Panel reflectors come
//   from CholeskyQR2 + Householder reconstruction (parallel over the p rows),
//   with a column-by-column Householder fallback for panels whose Gram
//   pivots collapse.  Panels are grouped into 512-column outer blocks: a
//   panel updates the rest of its outer block, and a finished outer block is
//   applied to all columns beyond it as one block reflector whose T is the UT
//   transform of the outer Y (exactly a product of the reflectors it holds).
//   Every block update
//     W = T^T (R_blk + Y^T C)   R_blk -= W   C -= Y W
//   runs on MFMA (bf16 operands with fp32 accumulation in MATH_BF16).
//   A chunk with r_in + p < n leaves an upper-trapezoidal R of r_in + p rows,
//   as torch.linalg.qr(mode="reduced") does for a wide chunk.
//
// finalize_R (triangular.py:386-421, scaled by activation_hooks.py:328-329):
//   the same fold with X = sqrt(lambda) I, using that X is upper triangular:
//   panel k only involves X rows [0, c1), i.e. (2/3) n^3 flops.
//
// Preconditioning (triangular.py:551-656, four solves):
//   Z = R^{-1} by a blocked triangular inverse (64 x 64 diagonal blocks
//   inverted in LDS, off-diagonal blocks by recursive doubling
//   Z12 = -Z11 R12 Z22 with batched MFMA GEMMs, log2(n/64) levels), then
//   nat = Z_G (Z_G^T grad) Z_X Z_X^T as four triangular MFMA products.
#include <algorithm>
#include <cstdint>
#include <map>
#include <mutex>
#include <cmath>

#include "gemm.h"
#include "kernels.h"
#include "linalg.h"
#include "lookahead.h"

namespace ifk {

#define RC(x)                 \
  do {                        \
    int _rc = (x);            \
    if (_rc) return _rc;      \
  } while (0)

// First-pass pivot threshold relative to the pivot's diagonal: panels with a
// smaller pivot (rank-deficient or kappa^2 beyond ~1e4) take the Householder
// fallback, so the second CholeskyQR pass always starts from a Q whose loss
// of orthogonality is far below its own 1/4 pivot threshold.
static constexpr float HR_TOL = 1e-4f;
static constexpr int64_t OUTER_B = 512;
// Outer block of the CholeskyQR path: a block's factorisation is a chain of
// latency-bound small kernels whose length grows slower than its width, so
// wider blocks cut the chain per column (and the far updates' read-modify-
// write of C per column), up to the 1024 the block Cholesky supports.
// Measured on the pair of factor updates of the 4096 -> 11008, p = 16384
// step: 512: 28.0 ms, 768: 26.0, 1024: 23.7.
static constexpr int64_t CQR_B = 1024;
// Workgroup cap of the far-column products on the helper stream: the far
// update is bound by HBM and runs beside the next block's factorisation,
// whose small kernels are bound by memory latency; capped, it leaves them CUs
// of their own.  192 measured best between 32 and uncapped on the
// 4096 -> 11008, p = 16384 step with 512-column CholeskyQR outer blocks (32:
// 69.7 ms, 128: 33.6, 192: 32.6, uncapped: 32.7 for the pair of factor
// updates) and again with 1024-column ones (64: 29.0, 96: 24.5, 128: 24.0,
// 192: 24.0, 256: 25.0).
static constexpr int FAR_MAX_WGS = 192;

static size_t split_floats(int64_t b, int64_t n) {
  size_t f = (size_t)64 * b * n;
  const size_t cap = (size_t)16 << 20;
  if (f > cap) f = cap;
  if (f < (size_t)64 * b * b) f = (size_t)64 * b * b;
  return f;
}

// ----------------------------------------------------------------------------
// Fold
// ----------------------------------------------------------------------------
static int trinv_core(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z,
                      int64_t ldz, int math, int safe, float* tmp, SplitScratch sp,
                      bool ut = false, int64_t w_stop = INT64_MAX);

struct FoldWs {
  int64_t B;      // outer block width the buffers are sized for (OUTER_B or CQR_B)
  float* C;       // n x p: the chunk, transposed (CT = C^T; see fold_core)
  bf16_t* Cb;     // n x p: RNE bf16 shadow of C for bf16 arithmetic (the rows of
                  // columns beyond the current outer block are kept current)
  float* Yo[2];   // p x OUTER_B: reflector X parts of an outer block (by block parity)
  bf16_t* Yob[2];   // bf16 copies of Yo, row-major and transposed (OUTER_B x p),
  bf16_t* YobT[2];  // for bf16 arithmetic (the products round their operands
                    // to bf16 anyway)
  float* Wpn;     // OUTER_B x OUTER_B: CT_cols Y + R_blk^T of the near columns
  float* Wpf;     // n x OUTER_B: ... of the far columns
  bf16_t* Wpnb;   // bf16 copies of Wpn, Wpf (bf16 arithmetic)
  bf16_t* Wpfb;
  float* Wn;      // OUTER_B x OUTER_B: W^T of the near columns (critical stream)
  float* Wf;      // n x OUTER_B: W^T of the far columns (helper stream)
  bf16_t* Wnb;
  bf16_t* Wfb;
  float* Q2;      // p x 64: X_p M1, or the fallback's reflectors
  float* part;    // per-slab Gram matrices of the panel kernels
  float* Gp;      // their sum: PANEL_MAX_CB blocks of 64 x 64
  float* NW;      // 64 x OUTER_B: N W of the panel
  float* U1;      // 64 x 64 panel scratch
  float* M1;
  float* Q1;
  float* N;
  float* Go;      // OUTER_B x OUTER_B: Gram of the outer reflectors (upper part)
  float* To[2];   // OUTER_B x OUTER_B: T of an outer block (by block parity)
  bf16_t* ToTb[2];  // its transpose in bf16 (bf16 arithmetic)
  float* ttmp;    // triangular-inverse scratch for To
  SplitScratch tsp;
  int* flag;
  SplitScratch split;   // split-K scratch of the critical stream
  SplitScratch split2;  // ... and of the helper stream
};

static void plan_fold(Arena& a, int64_t p, int64_t n, bool need_C, FoldWs& w,
                      int64_t B = OUTER_B) {
  const int64_t b = PANEL_B;
  w.B = B;
  w.C = need_C ? a.take<float>((size_t)p * n) : nullptr;
  w.Cb = need_C ? a.take<bf16_t>((size_t)p * n) : nullptr;
  for (int i = 0; i < 2; ++i) {
    w.Yo[i] = a.take<float>((size_t)p * B);
    w.Yob[i] = a.take<bf16_t>((size_t)p * B);
    w.YobT[i] = a.take<bf16_t>((size_t)p * B);
    w.To[i] = a.take<float>(B * B);
    w.ToTb[i] = a.take<bf16_t>(B * B);
  }
  w.Wpn = a.take<float>((size_t)B * B);
  w.Wpf = a.take<float>((size_t)B * n);
  w.Wpnb = a.take<bf16_t>((size_t)B * B);
  w.Wpfb = a.take<bf16_t>((size_t)B * n);
  w.Wn = a.take<float>((size_t)B * B);
  w.Wf = a.take<float>((size_t)B * n);
  w.Wnb = a.take<bf16_t>((size_t)B * B);
  w.Wfb = a.take<bf16_t>((size_t)B * n);
  w.Q2 = a.take<float>((size_t)p * b);
  w.part = a.take<float>((size_t)gram_slabs(p) * PANEL_MAX_CB * b * b);
  w.Gp = a.take<float>((size_t)PANEL_MAX_CB * b * b);
  w.NW = a.take<float>((size_t)b * B);
  w.U1 = a.take<float>(b * b);
  w.M1 = a.take<float>(b * b);
  w.Q1 = a.take<float>(b * b);
  w.N = a.take<float>(b * b);
  w.Go = a.take<float>(B * B);
  w.ttmp = a.take<float>((size_t)B * B / 2 + (size_t)TRINV_NB * TRINV_NB * 4);
  w.tsp.floats = split_floats(TRINV_NB, B);
  w.tsp.p = a.take<float>(w.tsp.floats);
  w.flag = a.take<int>(64);
  w.split.floats = split_floats(B, n);
  w.split.p = a.take<float>(w.split.floats);
  w.split2.floats = split_floats(B, n);
  w.split2.p = a.take<float>(w.split2.floats);
}

// Workspace of the block CholeskyQR path (cqr_pass1/2): CQR_B x CQR_B (1024 x
// 1024) factors of the outer block, the Cholesky's diagonal inverses, the
// block's tall operands in both layouts (pe x CQR_B row-major, and transposed
// CQR_B x pe with row stride ldq), fp32 or bf16 by the arithmetic, and -- by block parity,
// since a block's far update runs while the next block is factored -- the
// inverses M2 and N its outer update applies.
struct CqrWs {
  int64_t B;      // block width (CQR_B)
  float* G;       // G1, then G2
  float* U1;
  float* M1;      // U1^{-1}
  float* MT;      // M1^T (fp32 arithmetic), or its bf16 split hi | lo
  float* E;       // G2 - I (upper part)
  float* F[2];    // fixed-point iterates of U2 - I
  float* S;       // F^2, then U2 M2a (Newton step)
  float* M2a;     // first approximation of U2^{-1}
  float* Am;      // c M1 + U2
  float* Zd;      // CQR_B / 64 (16) x 64 x 64 diagonal-block inverses
  float* dref;
  float* Xc;      // X, pe x CQR_B (fp32 or bf16)
  float* Q2f;     // Q2 = X M1, pe x CQR_B fp32
  float* Q2T;     // Q2^T, CQR_B x pe (ld ldq; fp32 arithmetic)
  int64_t ldq;
  float* M2[2];   // U2^{-1} (fp32), and its transpose in bf16
  bf16_t* M2Tb[2];
  float* N[2];    // (c M1 + U2)^{-1} (fp32), and a row-major bf16 copy
  bf16_t* Nb[2];
  int* flag;      // set when a block needs the Householder path
};

static void plan_cqr(Arena& a, int64_t pe, CqrWs& q) {
  const int64_t B = CQR_B;
  q.B = B;
  const size_t pb = (size_t)(pe > 0 ? pe : 1) * B;
  q.G = a.take<float>(B * B);
  q.U1 = a.take<float>(B * B);
  q.M1 = a.take<float>(B * B);
  q.MT = a.take<float>(B * B);
  q.E = a.take<float>(B * B);
  q.F[0] = a.take<float>(B * B);
  q.F[1] = a.take<float>(B * B);
  q.S = a.take<float>(B * B);
  q.M2a = a.take<float>(B * B);
  q.Am = a.take<float>(B * B);
  q.Zd = a.take<float>((size_t)(B / 64) * 64 * 64);
  q.dref = a.take<float>(B);
  q.Xc = a.take<float>(pb);
  q.Q2f = a.take<float>(pb);
  q.ldq = (int64_t)align_up((size_t)(pe > 0 ? pe : 1), 8);
  q.Q2T = a.take<float>((size_t)B * q.ldq);
  for (int i = 0; i < 2; ++i) {
    q.M2[i] = a.take<float>(B * B);
    q.M2Tb[i] = a.take<bf16_t>(B * B);
    q.N[i] = a.take<float>(B * B);
    q.Nb[i] = a.take<bf16_t>(B * B);
  }
  q.flag = a.take<int>(64);
}

// One helper stream per (device, calling stream): folds issued on different
// streams (the two sides of a layer) keep independent far updates.
static std::mutex g_mu;
static std::map<std::pair<int, hipStream_t>, LookAhead*> g_la;

LookAhead* look_ahead(hipStream_t s, int* rc) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("tsqr_fold: hipGetDevice failed");
    *rc = IFK_ERR_HIP;
    return nullptr;
  }
  std::lock_guard<std::mutex> g(g_mu);
  LookAhead*& la = g_la[std::make_pair(dev, s)];
  if (!la) {
    LookAhead* x = new LookAhead();
    bool ok = hipStreamCreateWithFlags(&x->s2, hipStreamNonBlocking) == hipSuccess &&
              hipStreamCreateWithFlags(&x->s3, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreateWithFlags(&x->done, hipEventDisableTiming) == hipSuccess;
    for (int i = 0; i < 2 && ok; ++i)
      ok = hipEventCreateWithFlags(&x->ready[i], hipEventDisableTiming) == hipSuccess &&
           hipEventCreateWithFlags(&x->nearwp[i], hipEventDisableTiming) == hipSuccess &&
           hipEventCreateWithFlags(&x->fall[i], hipEventDisableTiming) == hipSuccess &&
           hipEventCreateWithFlags(&x->tready[i], hipEventDisableTiming) == hipSuccess &&
           hipEventCreateWithFlags(&x->aready[i], hipEventDisableTiming) == hipSuccess;
    if (!ok) {
      set_error("tsqr_fold: cannot create the helper stream or its events");
      *rc = IFK_ERR_HIP;
      return nullptr;
    }
    la = x;
  }
  *rc = IFK_OK;
  return la;
}

int look_ahead_release(hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("release_stream_state: hipGetDevice failed");
    return IFK_ERR_HIP;
  }
  std::lock_guard<std::mutex> g(g_mu);
  auto it = g_la.find(std::make_pair(dev, s));
  LookAhead* la = nullptr;
  if (it != g_la.end()) {
    la = it->second;
    g_la.erase(it);
  }
  if (!la) return IFK_OK;   // no helper streams were made for this stream
  bool ok = true;
  {
    std::lock_guard<std::mutex> l(la->mu);
    // the helpers' queued work, and the calling stream's waits on their
    // events, must finish before the streams and events go
    for (hipStream_t h : {la->s2, la->s3, s})
      if (h) ok = hipStreamSynchronize(h) == hipSuccess && ok;
    for (hipEvent_t e : la->col)
      if (e) ok = hipEventDestroy(e) == hipSuccess && ok;
    for (hipEvent_t e : {la->done, la->ready[0], la->ready[1], la->nearwp[0], la->nearwp[1],
                         la->fall[0], la->fall[1], la->tready[0], la->tready[1], la->aready[0],
                         la->aready[1]})
      if (e) ok = hipEventDestroy(e) == hipSuccess && ok;
    for (hipStream_t h : {la->s2, la->s3})
      if (h) ok = hipStreamDestroy(h) == hipSuccess && ok;
  }
  delete la;
  if (!ok) {
    set_error("release_stream_state: a helper stream or event could not be released");
    return IFK_ERR_HIP;
  }
  return IFK_OK;
}

int look_ahead_events(LookAhead* la, size_t n) {
  for (std::vector<hipEvent_t>* v : {&la->col}) {
    while (v->size() < n) {
      hipEvent_t e = nullptr;
      if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
        set_error("look-ahead: cannot create an event");
        return IFK_ERR_HIP;
      }
      v->push_back(e);
    }
  }
  return IFK_OK;
}


// T of outer block k (reflectors V = [I; Y] of columns [K0, K1), pe rows,
// buffers of parity k2).  The UT transform gives
//   T^{-1} = striu(V^T V) + diag(V^T V) / 2,   V^T V = I + Go,  Go = Y^T Y,
// and T is its triangular inverse (fp32): diagonal blocks straight from Go,
// the rest by block doubling.  In bf16 arithmetic Go reads the transposed
// bf16 copy of Y (both operands K-contiguous).
static int outer_prepare(hipStream_t s, int math, FoldWs& w, int k2, int64_t pe, int64_t ldt,
                         int64_t KB) {
  const int64_t B = OUTER_B;
  const bool bf = math == MATH_BF16;
  const MatRef YA = bf ? A_n(w.YobT[k2], DT_BF16, ldt) : A_t(w.Yo[k2], DT_F32, B);
  const MatRef YB = bf ? B_t(w.YobT[k2], DT_BF16, ldt) : B_n(w.Yo[k2], DT_F32, B);
  RC(gemm(s, math, KB, KB, pe, 1.0f, YA, YB, 0.0f, out_f32(w.Go, B), 1, w.split));
  RC(trinv_core(s, w.Go, DT_F32, B, KB, w.To[k2], B, MATH_F32, 0, w.ttmp, w.tsp, true));
  // T^T in bf16: the product W^T = Wp T then reads both operands K-contiguous
  return bf ? launch_transpose_cast(s, w.To[k2], B, KB, KB, w.ToTb[k2], DT_BF16, B) : IFK_OK;
}

// Apply outer block k to the columns [c_lo, c_hi) of C, i.e. the rows
// [c_lo, c_hi) of the transposed working matrix CT (ld ldc), in two halves:
//   outer_wp:     Wp = CT_cols Y + R_blk^T          (does not need T)
//   outer_finish: W^T = Wp T,  R_blk -= W,  CT_cols -= W^T Y^T
// The large products read K-contiguous operands only (CT or its bf16
// shadow, the transposed bf16 copy of Y).  Wp and W^T are nt x KB.
static int outer_wp(hipStream_t s, int math, FoldWs& w, int k2, float* CT, bf16_t* CTb,
                    int64_t ldc, int64_t pe, float* R, int64_t ldr, int64_t K0, int64_t K1,
                    int64_t c_lo, int64_t c_hi, float* Wp, bf16_t* Wpb, SplitScratch sp,
                    int max_wgs) {
  const int64_t B = OUTER_B, KB = K1 - K0, nt = c_hi - c_lo;
  if (nt <= 0) return IFK_OK;
  const bool bf = math == MATH_BF16;
  float* Cr = CT + c_lo * ldc;
  bf16_t* Crb = CTb ? CTb + c_lo * ldc : nullptr;   // bf16 shadow (bf16 arithmetic)
  RC(launch_transpose_to_f32(s, R + K0 * ldr + c_lo, DT_F32, ldr, KB, nt, Wp, KB));
  const MatRef CA = Crb ? A_n(Crb, DT_BF16, ldc) : A_n(Cr, DT_F32, ldc);
  const MatRef YB = bf ? B_t(w.YobT[k2], DT_BF16, ldc) : B_n(w.Yo[k2], DT_F32, B);
  return gemm(s, math, nt, KB, pe, 1.0f, CA, YB, 1.0f,
              bf ? out_both(Wp, KB, Wpb, KB) : out_f32(Wp, KB), 1, sp, max_wgs);
}

static int outer_finish(hipStream_t s, int math, FoldWs& w, int k2, float* CT, bf16_t* CTb,
                        int64_t ldc, int64_t pe, float* R, int64_t ldr, int64_t K0, int64_t K1,
                        int64_t c_lo, int64_t c_hi, const float* Wp, const bf16_t* Wpb, float* W,
                        bf16_t* Wb, SplitScratch sp, int max_wgs) {
  const int64_t B = OUTER_B, KB = K1 - K0, nt = c_hi - c_lo;
  if (nt <= 0) return IFK_OK;
  const bool bf = math == MATH_BF16;
  float* Rb = R + K0 * ldr + c_lo;
  float* Cr = CT + c_lo * ldc;
  bf16_t* Crb = CTb ? CTb + c_lo * ldc : nullptr;
  const MatRef WpA = bf ? A_n(Wpb, DT_BF16, KB) : A_n(Wp, DT_F32, KB);
  const MatRef TB = bf ? B_t(w.ToTb[k2], DT_BF16, B, TRI_UPPER) : B_n(w.To[k2], DT_F32, B, TRI_UPPER);
  RC(gemm(s, math, nt, KB, KB, 1.0f, WpA, TB, 0.0f, bf ? out_both(W, KB, Wb, KB) : out_f32(W, KB),
          1, sp, max_wgs));
  RC(launch_sub_transposed(s, Rb, ldr, W, KB, KB, nt));
  const MatRef WA = bf ? A_n(Wb, DT_BF16, KB) : A_n(W, DT_F32, KB);
  const MatRef YoBt = bf ? B_t(w.Yob[k2], DT_BF16, B) : B_t(w.Yo[k2], DT_F32, B);
  return gemm(s, math, nt, pe, KB, -1.0f, WA, YoBt, 1.0f,
              Crb ? out_both(Cr, ldc, Crb, ldc) : out_f32(Cr, ldc), 1, sp, max_wgs);
}

// Outer block [K0, K1) factored as a whole by CholeskyQR2, in place of its
// chain of 64-column panels.  P = [c I; X]: the block's rows of R are still
// the damping diagonal c I of the fused fold + finalize (only a block's own
// factorisation writes them) and its rows right of the block are still zero;
// X = C[:, K0:K1] (rows K0:K1 of CT, pe columns):
//   G1 = X^T X + c^2 I = U1^T U1,  M1 = U1^{-1},  Q2 = X M1
//   G2 = Q2^T Q2 + c^2 M1^T M1 = I + E = U2^T U2,  U2 = I + F
//   R_new = -U2 U1   (the sign the Householder form gives; R is
//                     sign-normalised at the end of the fold)
// G2 is close to the identity after the first pass, so U2 comes from the
// fixed point F = up(E - F^T F) (up = strict upper part + diag / 2; three
// sweeps from F = up(E)) instead of a second Cholesky, and M2 = U2^{-1} from
// (I - F)(I + F^2) (plus one Newton step in fp32 arithmetic).  A first-pass
// pivot below HR_TOL of its diagonal, or a last sweep that still moves F by
// more than 1e-6, sets q.flag: the block was too ill-conditioned for
// CholeskyQR and the factor must be recomputed by the panel path.
// The block reflector of the TPQRT form, Q^T = I - V T^T V^T with V = [I; Y],
// Y = X (c I - R_new)^{-1} and T = I - c R_new^{-1}, is never formed: applied
// to the columns right of the block ([0; C_rest], R rows still zero) it is
//   R_blk = -M2^T Q2^T C_rest,  C_rest -= Q2 N M2^T Q2^T C_rest,
//   N = (c M1 + U2)^{-1}
// (Y T = -X R_new^{-1} = Q2 M2 and Y = Q2 N), which outer_wp_q / outer_finish_q
// compute with Q2 in place of Y and the small factors M2, N in place of T.
// Every tall product reads K-contiguous operands: X and Q2 are kept in both
// layouts (the transposes are plain copies).
// bf16 arithmetic: X is read as bf16 (the shadow), Q2 = X (M1_hi + M1_lo)
// (the bf16 split of M1 keeps Q2 consistent with R_new to about 2^-17) is
// rounded to bf16 into the block's reflector store (row-major and
// transposed), and M2, N get bf16 copies; the 1024 x 1024 algebra is fp32.
// First pass, up to Q2 in the block's reflector store (all the outer update's
// S^T = CT_cols Q2 products need).
static int cqr_pass1(hipStream_t s, int math, FoldWs& w, CqrWs& q, int k2, float c,
                     const float* C, const bf16_t* Cb, int64_t ldc, int64_t pe, int64_t K0,
                     int64_t K1) {
  const int64_t B = q.B, KB = K1 - K0, ldq = q.ldq;
  const bool bf = math == MATH_BF16;
  const float* Xf = C + K0 * ldc;
  const bf16_t* Xb = Cb ? Cb + K0 * ldc : nullptr;
  // pass 1: G1 = X^T X + c^2 I = U1^T U1, M1 = U1^{-1}
  const MatRef XA = Xb ? A_n(Xb, DT_BF16, ldc) : A_n(Xf, DT_F32, ldc);
  const MatRef XB = Xb ? B_t(Xb, DT_BF16, ldc) : B_t(Xf, DT_F32, ldc);
  RC(gemm(s, math, KB, KB, pe, 1.0f, XA, XB, 0.0f, upper_part(out_f32(q.G, B)), 1, w.split));
  RC(launch_add_diag(s, q.G, B, KB, c * c));
  RC(launch_cholb(s, q.G, B, (int)KB, q.U1, B, q.Zd, q.dref, HR_TOL, q.flag, q.M1, B));
  // X in its pe x KB layout, then Q2 = X M1 (pe x KB) into the reflector store
  if (Xb) RC(launch_transpose_bf16(s, Xb, ldc, KB, pe, (bf16_t*)q.Xc, B));
  else RC(launch_transpose_cast(s, Xf, ldc, KB, pe, q.Xc, bf ? DT_BF16 : DT_F32, B));
  if (bf) {
    bf16_t* MTh = (bf16_t*)q.MT;
    bf16_t* MTl = MTh + B * B;
    RC(launch_split_bf16(s, q.M1, B, KB, KB, MTh, MTl, B, true));
    RC(gemm(s, MATH_BF16, pe, KB, KB, 1.0f, A_n(q.Xc, DT_BF16, B),
            B_t(MTh, DT_BF16, B, TRI_UPPER), 0.0f, out_f32(q.Q2f, B), 1, w.split));
    RC(gemm(s, MATH_BF16, pe, KB, KB, 1.0f, A_n(q.Xc, DT_BF16, B),
            B_t(MTl, DT_BF16, B, TRI_UPPER), 1.0f, out_both(q.Q2f, B, w.Yob[k2], B), 1,
            w.split));
    return launch_transpose_bf16(s, w.Yob[k2], B, pe, KB, w.YobT[k2], ldc);
  }
  RC(launch_transpose_cast(s, q.M1, B, KB, KB, q.MT, DT_F32, B));
  RC(gemm(s, MATH_F32, pe, KB, KB, 1.0f, A_n(q.Xc, DT_F32, B), B_t(q.MT, DT_F32, B, TRI_UPPER),
          0.0f, out_f32(w.Yo[k2], B), 1, w.split));
  return launch_transpose_cast(s, w.Yo[k2], B, pe, KB, q.Q2T, DT_F32, ldq);
}

// Second pass from the Q2 of cqr_pass1: R_new into R, and for an outer block
// the small factors M2 and N of its outer update.
static int cqr_pass2(hipStream_t s, int math, FoldWs& w, CqrWs& q, int k2, float c,
                     int64_t ldc, int64_t pe, float* R, int64_t ldr, int64_t K0, int64_t K1,
                     bool outer) {
  const int64_t B = q.B, KB = K1 - K0, ldq = q.ldq;
  const bool bf = math == MATH_BF16;
  // G2 = Q2^T Q2
  if (bf)
    RC(gemm(s, MATH_BF16, KB, KB, pe, 1.0f, A_n(w.YobT[k2], DT_BF16, ldc),
            B_t(w.YobT[k2], DT_BF16, ldc), 0.0f, upper_part(out_f32(q.G, B)), 1, w.split));
  else
    RC(gemm(s, MATH_F32, KB, KB, pe, 1.0f, A_n(q.Q2T, DT_F32, ldq), B_t(q.Q2T, DT_F32, ldq), 0.0f,
            upper_part(out_f32(q.G, B)), 1, w.split));
  SqmmArgs a;
  a.M = a.N = a.K = KB;
  a.ldo = B;
  // E = G2 + c^2 M1^T M1 - I (upper part), and F = up(E)
  {
    SqmmArgs e = a;
    e.A = q.M1, e.lda = B, e.ta = 1, e.tria = TRI_LOWER;
    e.B = q.M1, e.ldb = B, e.trib = TRI_UPPER;
    e.alpha = c * c;
    e.C1 = q.G, e.ld1 = B, e.beta1 = 1.0f;
    e.gamma = -1.0f;
    e.epi = SQ_TRIU;
    e.out = q.E;
    e.out2 = q.F[0];
    RC(launch_sqmm(s, &e));
  }
  // U2 = I + F: sweeps F <- up(E - F^T F), the last one tested.  Each sweep
  // cuts the error by about 2 ||F||; bf16 arithmetic needs F to about 1e-6
  // (two sweeps, the last moving no entry by more than 1e-4), fp32 arithmetic
  // to fp32 rounding (three, 1e-6).
  const int sweeps = bf ? 2 : 3;
  int cur = 0;
  for (int it = 0; it < sweeps; ++it, cur ^= 1) {
    SqmmArgs f = a;
    f.A = q.F[cur], f.lda = B, f.ta = 1, f.tria = TRI_LOWER;
    f.B = q.F[cur], f.ldb = B, f.trib = TRI_UPPER;
    f.alpha = -1.0f;
    f.C1 = q.E, f.ld1 = B, f.beta1 = 1.0f;
    f.epi = SQ_UP;
    f.out = q.F[cur ^ 1];
    if (it == sweeps - 1) f.prev = q.F[cur], f.tol = bf ? 1e-4f : 1e-6f, f.flag = q.flag;
    RC(launch_sqmm(s, &f));
  }
  const float* F = q.F[cur];
  // in one launch: R_new = -U2 U1 = -(U1 + F U1); M2 = U2^{-1} = I - F + F^2
  // (the dropped -F^3 is below 1e-9 for the F of bf16 rounding noise and far
  // below the bf16 rounding of M2's uses; fp32 arithmetic forms F^2 here and
  // refines below); and c M1 + U2, whose inverse is N
  SqmmArgs t[3];
  t[0] = a;
  t[0].A = F, t[0].lda = B, t[0].tria = TRI_UPPER;
  t[0].B = q.U1, t[0].ldb = B, t[0].trib = TRI_UPPER;
  t[0].alpha = -1.0f;
  t[0].C1 = q.U1, t[0].ld1 = B, t[0].beta1 = -1.0f;
  t[0].epi = SQ_TRIU;
  t[0].out = R + K0 * ldr + K0, t[0].ldo = ldr;
  t[1] = a;
  t[1].A = F, t[1].lda = B, t[1].tria = TRI_UPPER;
  t[1].B = F, t[1].ldb = B, t[1].trib = TRI_UPPER;
  t[1].epi = SQ_TRIU;
  if (bf) {
    t[1].C1 = F, t[1].ld1 = B, t[1].beta1 = -1.0f;
    t[1].gamma = 1.0f;
    t[1].out = q.M2[k2];
    t[1].outb = q.M2Tb[k2], t[1].ldob = B, t[1].outb_t = 1;
  } else {
    t[1].out = q.S;
  }
  t[2] = a;
  t[2].alpha = 0.0f;
  t[2].C1 = q.M1, t[2].ld1 = B, t[2].beta1 = c;
  t[2].C2 = F, t[2].ld2 = B, t[2].beta2 = 1.0f;
  t[2].gamma = 1.0f;
  t[2].epi = SQ_TRIU;
  t[2].out = q.Am;
  RC(launch_sqmm(s, t, outer ? 3 : 1));
  if (!outer) return IFK_OK;
  // fp32 arithmetic: M2a = (I - F)(I + F^2) = I + F^2 - F - F F^2, then one
  // Newton step M2 = M2a (2 I - U2 M2a)
  if (!bf) {
    {
      SqmmArgs m = a;
      m.A = F, m.lda = B, m.tria = TRI_UPPER;
      m.B = q.S, m.ldb = B, m.trib = TRI_UPPER;
      m.alpha = -1.0f;
      m.C1 = q.S, m.ld1 = B, m.beta1 = 1.0f;
      m.C2 = F, m.ld2 = B, m.beta2 = -1.0f;
      m.gamma = 1.0f;
      m.epi = SQ_TRIU;
      m.out = q.M2a;
      RC(launch_sqmm(s, &m));
    }
    SqmmArgs m = a;
    m.A = F, m.lda = B, m.tria = TRI_UPPER;
    m.B = q.M2a, m.ldb = B, m.trib = TRI_UPPER;
    m.C1 = q.M2a, m.ld1 = B, m.beta1 = 1.0f;
    m.epi = SQ_TRIU;
    m.out = q.S;   // U2 M2a
    RC(launch_sqmm(s, &m));
    m.A = q.M2a;
    m.B = q.S;
    m.alpha = -1.0f;
    m.beta1 = 2.0f;
    m.out = q.M2[k2];
    RC(launch_sqmm(s, &m));
  }
  // N = (c M1 + U2)^{-1}
  RC(trinv_core(s, q.Am, DT_F32, B, KB, q.N[k2], B, MATH_F32, 0, w.ttmp, w.tsp));
  return bf ? launch_cast(s, q.N[k2], B, KB, KB, q.Nb[k2], DT_BF16, B) : IFK_OK;
}

// Outer update of a CholeskyQR'd block (see cqr_pass1/2) on the columns
// [c_lo, c_hi) of C, i.e. the rows of CT, in two halves:
//   outer_wp_q:     S^T = CT_cols Q2
//   outer_finish_q: S2^T = S^T M2,  R_blk -= S2,  Z^T = S2^T N^T (into Wp),
//                   CT_cols -= Z^T Q2^T
static int outer_wp_q(hipStream_t s, int math, FoldWs& w, int k2, float* CT, bf16_t* CTb,
                      int64_t ldc, int64_t pe, int64_t KB, int64_t c_lo, int64_t c_hi, float* Wp,
                      bf16_t* Wpb, SplitScratch sp, int max_wgs) {
  const int64_t B = w.B, nt = c_hi - c_lo;
  if (nt <= 0) return IFK_OK;
  const bool bf = math == MATH_BF16;
  const MatRef CA = CTb ? A_n(CTb + c_lo * ldc, DT_BF16, ldc) : A_n(CT + c_lo * ldc, DT_F32, ldc);
  const MatRef QB = bf ? B_t(w.YobT[k2], DT_BF16, ldc) : B_n(w.Yo[k2], DT_F32, B);
  return gemm(s, math, nt, KB, pe, 1.0f, CA, QB, 0.0f,
              bf ? out_both(Wp, KB, Wpb, KB) : out_f32(Wp, KB), 1, sp, max_wgs);
}

static int outer_finish_q(hipStream_t s, int math, FoldWs& w, CqrWs& q, int k2, float* CT,
                          bf16_t* CTb, int64_t ldc, int64_t pe, float* R, int64_t ldr, int64_t K0,
                          int64_t K1, int64_t c_lo, int64_t c_hi, float* Wp, bf16_t* Wpb,
                          float* W, bf16_t* Wb, SplitScratch sp, int max_wgs) {
  const int64_t B = w.B, KB = K1 - K0, nt = c_hi - c_lo;
  if (nt <= 0) return IFK_OK;
  const bool bf = math == MATH_BF16;
  float* Cr = CT + c_lo * ldc;
  bf16_t* Crb = CTb ? CTb + c_lo * ldc : nullptr;
  const MatRef SA = bf ? A_n(Wpb, DT_BF16, KB) : A_n(Wp, DT_F32, KB);
  const MatRef MB = bf ? B_t(q.M2Tb[k2], DT_BF16, B, TRI_UPPER)
                       : B_n(q.M2[k2], DT_F32, B, TRI_UPPER);
  RC(gemm(s, math, nt, KB, KB, 1.0f, SA, MB, 0.0f, bf ? out_both(W, KB, Wb, KB) : out_f32(W, KB),
          1, sp, max_wgs));
  RC(launch_sub_transposed(s, R + K0 * ldr + c_lo, ldr, W, KB, KB, nt));
  const MatRef WA = bf ? A_n(Wb, DT_BF16, KB) : A_n(W, DT_F32, KB);
  const MatRef NB = bf ? B_t(q.Nb[k2], DT_BF16, B, TRI_LOWER)
                       : B_t(q.N[k2], DT_F32, B, TRI_LOWER);
  RC(gemm(s, math, nt, KB, KB, 1.0f, WA, NB, 0.0f, bf ? out_bf16(Wpb, KB) : out_f32(Wp, KB), 1, sp,
          max_wgs));
  const MatRef ZA = bf ? A_n(Wpb, DT_BF16, KB) : A_n(Wp, DT_F32, KB);
  const MatRef QBt = bf ? B_t(w.Yob[k2], DT_BF16, B) : B_t(w.Yo[k2], DT_F32, B);
  return gemm(s, math, nt, pe, KB, -1.0f, ZA, QBt, 1.0f,
              Crb ? out_both(Cr, ldc, Crb, ldc) : out_f32(Cr, ldc), 1, sp, max_wgs);
}

// Core of the fold on the transposed fp32 working copy CT = C^T (n x p, row
// stride ldc; a panel X_p = C[:, c0:c1] is the contiguous row block
// CT[c0:c1, :]).  R rows [0, r_new) receive the result.  Two-level blocking:
// 64-column panels inside 512-column outer blocks; a panel's reflectors
// update only the rest of its outer block, and each finished outer block is
// applied to the columns beyond it as one block reflector.  Look-ahead: of
// that application only the T-dependent half for the next outer block's
// columns stays on the critical stream s; the rest runs on the device's
// helper stream and overlaps the next block's panels (which are latency-bound
// on a few CUs).  The application's large product CT_cols Y does not need T,
// so the helper forms it for every column beyond the block (the next block's
// first) as soon as the block's reflectors are written, while s forms T.
// Buffers a far update still reads are double buffered by block parity, and
// events order
//   panels(k) -> helper Wp(k);  T(k) on s -> helper finish(k);
//   helper near Wp(k) (after everything earlier on the helper) -> near(k);
//   far(k - 2) -> panels(k);  far(last) -> end of fold.
// With x_tri, C is upper triangular and a panel ending at column c1
// involves C rows [0, c1).
// With cq, every outer block is factored by cqr_pass1/2; R's rows are then
// expected to hold c I on entry (cq_c), as fold_finalize sets them.
static int fold_core(hipStream_t s, float* C, int64_t ldc, int64_t p, int64_t n, float* R,
                     int64_t ldr, int64_t r_new, bool x_tri, int math, FoldWs& w,
                     CqrWs* cq = nullptr, float cq_c = 0.0f) {
  const int64_t B = w.B;
  int rc = IFK_OK;
  LookAhead* la = nullptr;
  if (std::min<int64_t>(B, r_new) + B < n) {  // some block has columns beyond the next one
    la = look_ahead(s, &rc);
    if (!la) return rc;
  }
  std::unique_lock<std::mutex> lock;
  if (la) lock = std::unique_lock<std::mutex>(la->mu);
  const bool bf = math == MATH_BF16;
  // bf16 arithmetic: the outer-block products read a bf16 shadow of C (the
  // exact values their operand staging would round to), which the C updates
  // keep current; it is seeded here once
  bf16_t* Cb = (bf && w.Cb && std::min<int64_t>(B, r_new) < n) ? w.Cb : nullptr;
  if (Cb) RC(launch_cast(s, C, ldc, n, p, Cb, DT_BF16, ldc));
  bool fall_pending[2] = {false, false};   // a far update still reads parity buffers
  int a_prev = -1;   // parity of the previous block's far part A event, if recorded
  int k = 0;
  for (int64_t K0 = 0; K0 < r_new; K0 += B, ++k) {
    const int k2 = k & 1;
    const int64_t K1 = std::min<int64_t>(K0 + B, r_new);
    const int64_t KB = K1 - K0;
    const int64_t pe_o = x_tri ? std::min<int64_t>(p, K1) : p;
    const bool outer = K1 < n;   // the block is applied to columns beyond it
    // block k - 2's far update reads this parity's reflector store
    if (fall_pending[k2]) {
      HIPRC(hipStreamWaitEvent(s, la->fall[k2], 0), "tsqr_fold: stream wait failed");
      fall_pending[k2] = false;
    }
    if (x_tri) {
      RC(launch_zero(s, w.Yo[k2], B, pe_o, KB));
      if (bf) RC(launch_zero_bf16(s, w.Yob[k2], B, pe_o, KB));
      if (bf && outer) RC(launch_zero_bf16(s, w.YobT[k2], ldc, KB, pe_o));
    }
    if (cq) {
      RC(cqr_pass1(s, math, w, *cq, k2, cq_c, C, Cb, ldc, pe_o, K0, K1));
      if (!outer) RC(cqr_pass2(s, math, w, *cq, k2, cq_c, ldc, pe_o, R, ldr, K0, K1, false));
    }
    for (int64_t c0 = K0; c0 < K1 && !cq; c0 += PANEL_B) {
      const int bk = (int)std::min<int64_t>(PANEL_B, K1 - c0);
      const int64_t c1 = c0 + bk;
      const int nr = (int)(K1 - c1);
      const int64_t pe = x_tri ? std::min<int64_t>(p, c1) : p;
      float* Ptop = R + c0 * ldr + c0;
      float* XpT = C + c0 * ldc;
      int ncb;
      // pass 1: G1 = X_p^T X_p (+ P_top^T P_top), U1, M1 -- or the fallback
      RC(launch_gram(s, XpT, ldc, bk, true, nullptr, 0, 0, XpT, ldc, bk, pe, w.part, w.Gp, &ncb));
      RC(launch_panel_hr_a(s, w.Gp, Ptop, ldr, bk, HR_TOL, w.U1, w.M1, w.Q1, w.flag));
      // pass 2: Q2 = X_p M1 (or the fallback), G2 = Q2^T Q2 and Q2^T C_rest in one sweep
      RC(launch_apply_m(s, XpT, ldc, pe, bk, w.M1, w.Q2, Ptop, ldr, w.flag));
      RC(launch_gram(s, w.Q2, PANEL_B, PANEL_B, false, w.Q2, PANEL_B, PANEL_B, C + c1 * ldc, ldc,
                     nr, pe, w.part, w.Gp, &ncb));
      // reconstruction, R_new, and the rest of the outer block's R rows
      RC(launch_panel_hrw(s, w.Gp, ncb, w.Q1, w.U1, bk, w.N, Ptop, ldr, nr, w.NW, OUTER_B,
                          w.flag));
      // C_rest and Y into the outer store
      RC(launch_panel_update(s, w.Q2, pe, bk, w.N, w.Yo[k2] + (c0 - K0), OUTER_B,
                             bf ? w.Yob[k2] + (c0 - K0) : nullptr,
                             (bf && outer) ? w.YobT[k2] + (c0 - K0) * ldc : nullptr, ldc, w.NW,
                             OUTER_B, C + c1 * ldc, ldc, nr));
    }
    if (!outer) continue;
    const int64_t near_hi = std::min<int64_t>(K1 + B, n);
    const bool far = la && near_hi < n;
    const int64_t mid = std::min<int64_t>(near_hi + B, n);
    const int64_t ntA = mid - near_hi;   // far part A: the block after next
    if (cq) {
      // the helper forms S^T = CT_cols Q2 for far part A and the rest while s
      // runs the second pass; once M2 and N are there it finishes part A (the
      // next block's near columns), then the rest.  s applies the block to
      // its near columns itself, after the previous block's part A only (not
      // behind that block's whole far update on the helper).
      if (la) {
        const int64_t lo[2] = {near_hi, mid}, hi[2] = {mid, n};
        float* Wp[2] = {w.Wpf, w.Wpf + ntA * KB};
        bf16_t* Wpb[2] = {w.Wpfb, w.Wpfb + ntA * KB};
        if (far) {
          HIPRC(hipEventRecord(la->ready[k2], s), "tsqr_fold: event record failed");
          HIPRC(hipStreamWaitEvent(la->s2, la->ready[k2], 0), "tsqr_fold: stream wait failed");
          for (int part = 0; part < 2; ++part)
            RC(outer_wp_q(la->s2, math, w, k2, C, Cb, ldc, pe_o, KB, lo[part], hi[part],
                          Wp[part], Wpb[part], w.split2, FAR_MAX_WGS));
        }
        RC(cqr_pass2(s, math, w, *cq, k2, cq_c, ldc, pe_o, R, ldr, K0, K1, true));
        if (far) {
          HIPRC(hipEventRecord(la->tready[k2], s), "tsqr_fold: event record failed");
          HIPRC(hipStreamWaitEvent(la->s2, la->tready[k2], 0), "tsqr_fold: stream wait failed");
          RC(outer_finish_q(la->s2, math, w, *cq, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, lo[0],
                            hi[0], Wp[0], Wpb[0], w.Wf, w.Wfb, w.split2, FAR_MAX_WGS));
          HIPRC(hipEventRecord(la->aready[k2], la->s2), "tsqr_fold: event record failed");
          RC(outer_finish_q(la->s2, math, w, *cq, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, lo[1],
                            hi[1], Wp[1], Wpb[1], w.Wf, w.Wfb, w.split2, FAR_MAX_WGS));
          HIPRC(hipEventRecord(la->fall[k2], la->s2), "tsqr_fold: event record failed");
          fall_pending[k2] = true;
          HIPRC(hipEventRecord(la->done, la->s2), "tsqr_fold: event record failed");
        }
        if (a_prev >= 0)
          HIPRC(hipStreamWaitEvent(s, la->aready[a_prev], 0), "tsqr_fold: stream wait failed");
        a_prev = far ? k2 : -1;
        RC(outer_wp_q(s, math, w, k2, C, Cb, ldc, pe_o, KB, K1, near_hi, w.Wpn, w.Wpnb, w.split,
                      0));
        RC(outer_finish_q(s, math, w, *cq, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, K1, near_hi,
                          w.Wpn, w.Wpnb, w.Wn, w.Wnb, w.split, 0));
      } else {
        RC(cqr_pass2(s, math, w, *cq, k2, cq_c, ldc, pe_o, R, ldr, K0, K1, true));
        RC(outer_wp_q(s, math, w, k2, C, Cb, ldc, pe_o, KB, K1, n, w.Wpf, w.Wpfb, w.split, 0));
        RC(outer_finish_q(s, math, w, *cq, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, K1, n, w.Wpf,
                          w.Wpfb, w.Wf, w.Wfb, w.split, 0));
      }
      continue;
    }
    if (la) {
      // the T-independent half on the helper stream, from the moment the
      // block's reflectors are written, while s forms T: the near columns
      // first (s takes them back), then far part A and the rest beyond
      HIPRC(hipEventRecord(la->ready[k2], s), "tsqr_fold: event record failed");
      HIPRC(hipStreamWaitEvent(la->s2, la->ready[k2], 0), "tsqr_fold: stream wait failed");
      RC(outer_wp(la->s2, math, w, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, K1, near_hi, w.Wpn,
                  w.Wpnb, w.split2, 0));
      HIPRC(hipEventRecord(la->nearwp[k2], la->s2), "tsqr_fold: event record failed");
      if (far) {
        RC(outer_wp(la->s2, math, w, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, near_hi, mid, w.Wpf,
                    w.Wpfb, w.split2, FAR_MAX_WGS));
        RC(outer_wp(la->s2, math, w, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, mid, n,
                    w.Wpf + ntA * KB, w.Wpfb + ntA * KB, w.split2, FAR_MAX_WGS));
      }
    }
    RC(outer_prepare(s, math, w, k2, pe_o, ldc, KB));
    if (far) {
      // the T-dependent half of the far columns: part A first (the next
      // block's near columns wait for it), then the rest
      HIPRC(hipEventRecord(la->tready[k2], s), "tsqr_fold: event record failed");
      HIPRC(hipStreamWaitEvent(la->s2, la->tready[k2], 0), "tsqr_fold: stream wait failed");
      RC(outer_finish(la->s2, math, w, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, near_hi, mid, w.Wpf,
                      w.Wpfb, w.Wf, w.Wfb, w.split2, FAR_MAX_WGS));
      RC(outer_finish(la->s2, math, w, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, mid, n,
                      w.Wpf + ntA * KB, w.Wpfb + ntA * KB, w.Wf, w.Wfb, w.split2, FAR_MAX_WGS));
      HIPRC(hipEventRecord(la->fall[k2], la->s2), "tsqr_fold: event record failed");
      fall_pending[k2] = true;
      HIPRC(hipEventRecord(la->done, la->s2), "tsqr_fold: event record failed");
    }
    if (la) {
      // the near Wp, and with it every earlier far update (the previous
      // block's part A covers these columns)
      HIPRC(hipStreamWaitEvent(s, la->nearwp[k2], 0), "tsqr_fold: stream wait failed");
      RC(outer_finish(s, math, w, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, K1, near_hi, w.Wpn,
                      w.Wpnb, w.Wn, w.Wnb, w.split, 0));
    } else {
      RC(outer_wp(s, math, w, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, K1, n, w.Wpf, w.Wpfb, w.split,
                  0));
      RC(outer_finish(s, math, w, k2, C, Cb, ldc, pe_o, R, ldr, K0, K1, K1, n, w.Wpf, w.Wpfb, w.Wf,
                      w.Wfb, w.split, 0));
    }
  }
  if (la) HIPRC(hipStreamWaitEvent(s, la->done, 0), "tsqr_fold: stream wait failed");
  return launch_sign_normalize(s, R, ldr, r_new, n);
}

size_t fold_ws(int64_t p, int64_t n) {
  Arena a(nullptr, 0);
  FoldWs w;
  plan_fold(a, p, n, true, w);
  return a.used;
}

static int check_ws(const Arena& a, const char* what) {
  if (a.overflow) {
    set_error(std::string(what) + ": workspace too small");
    return IFK_ERR_WORKSPACE;
  }
  return IFK_OK;
}

int fold(hipStream_t s, const void* X, int xdt, int64_t p, int64_t n, int64_t ldx, float* R,
         int64_t ldr, int64_t r_in, int math, void* ws, size_t ws_bytes, int64_t* r_out) {
  if (n < 1 || p < 0 || ldr < n || r_in < 0 || r_in > n || (p > 0 && ldx < n) || !R ||
      (p > 0 && !X) || (xdt != DT_F32 && xdt != DT_BF16)) {
    set_error("tsqr_fold: invalid arguments");
    return IFK_ERR_INVALID;
  }
  if (p == 0) {
    if (r_out) *r_out = r_in;
    return IFK_OK;
  }
  const int64_t r_new = std::min<int64_t>(r_in + p, n);
  Arena a(ws, ws_bytes);
  FoldWs w;
  plan_fold(a, p, n, true, w);
  RC(check_ws(a, "tsqr_fold"));
  RC(launch_zero_rows(s, R, ldr, r_in, n, n));
  RC(launch_transpose_to_f32(s, X, xdt, ldx, p, n, w.C, p));
  RC(fold_core(s, w.C, p, p, n, R, ldr, r_new, false, math, w));
  if (r_out) *r_out = r_new;
  return IFK_OK;
}

// ----------------------------------------------------------------------------
// Finalize
// ----------------------------------------------------------------------------
static void plan_finalize(Arena& a, int64_t n, float** Rw, FoldWs& w) {
  *Rw = a.take<float>((size_t)n * n);
  plan_fold(a, n, n, true, w);
}

size_t finalize_ws(int64_t n) {
  Arena a(nullptr, 0);
  float* Rw;
  FoldWs w;
  plan_finalize(a, n, &Rw, w);
  return a.used;
}

int finalize(hipStream_t s, const float* R_in, int64_t ldr_in, int64_t n, float scale,
             float damping, void* out, int odt, int64_t ldo, int math, int* finite, void* ws,
             size_t ws_bytes) {
  if (n < 1 || ldr_in < n || ldo < n || !R_in || !out || !(damping >= 0.0f) ||
      (odt != DT_F32 && odt != DT_BF16)) {
    set_error("finalize: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float* Rw;
  FoldWs w;
  plan_finalize(a, n, &Rw, w);
  RC(check_ws(a, "finalize"));
  RC(launch_copy_upper(s, R_in, ldr_in, n, scale, Rw, n));
  RC(launch_set_diag(s, w.C, n, n, std::sqrt(damping)));
  RC(fold_core(s, w.C, n, n, n, Rw, n, n, true, math, w));
  if (finite) RC(launch_fill_int(s, finite, 1, 1));
  return launch_cast_upper(s, Rw, n, n, out, odt, ldo, finite);
}

// ----------------------------------------------------------------------------
// Fold and finalize in one factorisation
// ----------------------------------------------------------------------------
// The damped factor of the rows already folded (R_in, r_in rows) plus a
// chunk X is the R of [scale R_in; scale X; sqrt(damping) I], which is
// scale times the R of [R_in; X; c I] with c = sqrt(damping) / scale.  The
// triangular c I is the top block of one TPQRT fold whose working matrix is
// [R_in; X] (r_in + p rows): a single dependent panel chain instead of a fold
// followed by a finalize.
static void plan_fold_finalize(Arena& a, int64_t pe, int64_t n, float** Rw, FoldWs& w) {
  *Rw = a.take<float>((size_t)n * n);
  plan_fold(a, pe, n, true, w);
}

size_t fold_finalize_ws(int64_t p, int64_t n, int64_t r_in) {
  Arena a(nullptr, 0);
  float* Rw;
  FoldWs w;
  plan_fold_finalize(a, r_in + p, n, &Rw, w);
  return a.used;
}

int fold_finalize(hipStream_t s, const void* X, int xdt, int64_t p, int64_t n, int64_t ldx,
                  const float* R_in, int64_t ldr, int64_t r_in, float scale, float damping,
                  void* out, int odt, int64_t ldo, int math, int* finite, void* ws,
                  size_t ws_bytes) {
  if (n < 1 || p < 0 || r_in < 0 || r_in > n || (p > 0 && (!X || ldx < n)) ||
      (r_in > 0 && (!R_in || ldr < n)) || !out || ldo < n || !(scale > 0.0f) ||
      !(damping >= 0.0f) || (xdt != DT_F32 && xdt != DT_BF16) ||
      (odt != DT_F32 && odt != DT_BF16)) {
    set_error("fold_finalize: invalid arguments");
    return IFK_ERR_INVALID;
  }
  const int64_t pe = r_in + p;
  if (!(damping > 0.0f) && pe < n) {
    set_error("fold_finalize: fewer rows than columns and no damping (the factor is not square)");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float* Rw;
  FoldWs w;
  plan_fold_finalize(a, pe, n, &Rw, w);
  RC(check_ws(a, "fold_finalize"));
  RC(launch_set_diag(s, Rw, n, n, std::sqrt(damping) / scale));
  if (r_in > 0) RC(launch_transpose_to_f32(s, R_in, DT_F32, ldr, r_in, n, w.C, pe, true));
  if (p > 0) RC(launch_transpose_to_f32(s, X, xdt, ldx, p, n, w.C + r_in, pe));
  if (pe > 0) {
    RC(fold_core(s, w.C, pe, pe, n, Rw, n, n, false, math, w));
  } else {
    RC(launch_sign_normalize(s, Rw, n, n, n));
  }
  if (finite) RC(launch_fill_int(s, finite, 1, 1));
  return launch_cast_upper(s, Rw, n, n, out, odt, ldo, finite, scale);
}

// The same factor with every outer block factored by cqr_block instead of
// its panel chain.  *status: 1 = the factor is finite, 0 = not finite, 2 =
// some block was too ill-conditioned for CholeskyQR (the output is then
// meaningless and the caller recomputes it with fold_finalize).
static void plan_fold_finalize_cqr(Arena& a, int64_t pe, int64_t n, float** Rw, FoldWs& w,
                                   CqrWs& q) {
  *Rw = a.take<float>((size_t)n * n);
  plan_fold(a, pe, n, true, w, CQR_B);
  plan_cqr(a, pe, q);
}

size_t fold_finalize_cqr_ws(int64_t p, int64_t n, int64_t r_in) {
  Arena a(nullptr, 0);
  float* Rw;
  FoldWs w;
  CqrWs q;
  plan_fold_finalize_cqr(a, r_in + p, n, &Rw, w, q);
  return a.used;
}

int fold_finalize_cqr(hipStream_t s, const void* X, int xdt, int64_t p, int64_t n, int64_t ldx,
                      const float* R_in, int64_t ldr, int64_t r_in, float scale, float damping,
                      void* out, int odt, int64_t ldo, int math, int* status, void* ws,
                      size_t ws_bytes) {
  if (n < 1 || p < 0 || r_in < 0 || r_in > n || (p > 0 && (!X || ldx < n)) ||
      (r_in > 0 && (!R_in || ldr < n)) || !out || ldo < n || !(scale > 0.0f) ||
      !(damping >= 0.0f) || (xdt != DT_F32 && xdt != DT_BF16) ||
      (odt != DT_F32 && odt != DT_BF16) || !status) {
    set_error("fold_finalize_cqr: invalid arguments");
    return IFK_ERR_INVALID;
  }
  const int64_t pe = r_in + p;
  if (!(damping > 0.0f) && pe < n) {
    set_error("fold_finalize_cqr: fewer rows than columns and no damping (the factor is not square)");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float* Rw;
  FoldWs w;
  CqrWs q;
  plan_fold_finalize_cqr(a, pe, n, &Rw, w, q);
  RC(check_ws(a, "fold_finalize_cqr"));
  RC(launch_fill_int(s, q.flag, 0, 1));
  RC(launch_set_diag(s, Rw, n, n, std::sqrt(damping) / scale));
  if (r_in > 0) RC(launch_transpose_to_f32(s, R_in, DT_F32, ldr, r_in, n, w.C, pe, true));
  if (p > 0) RC(launch_transpose_to_f32(s, X, xdt, ldx, p, n, w.C + r_in, pe));
  if (pe > 0) {
    RC(fold_core(s, w.C, pe, pe, n, Rw, n, n, false, math, w, &q, std::sqrt(damping) / scale));
  } else {
    RC(launch_sign_normalize(s, Rw, n, n, n));
  }
  RC(launch_fill_int(s, status, 1, 1));
  RC(launch_cast_upper(s, Rw, n, n, out, odt, ldo, status, scale));
  return launch_status_merge(s, status, q.flag);
}

// ----------------------------------------------------------------------------
// Triangular inverse
// ----------------------------------------------------------------------------
static void plan_trinv(Arena& a, int64_t n, float** tmp, SplitScratch* sp) {
  *tmp = a.take<float>((size_t)n * n / 2 + (size_t)TRINV_NB * TRINV_NB * 4);
  sp->floats = split_floats(TRINV_NB, n);
  sp->p = a.take<float>(sp->floats);
}

// ... plus the bf16 copies of Z used by bf16 arithmetic: transposed, then
// row-major (2 n^2 elements from zt)
static void plan_trinv(Arena& a, int64_t n, float** tmp, bf16_t** zt, SplitScratch* sp) {
  plan_trinv(a, n, tmp, sp);
  *zt = a.take<bf16_t>((size_t)n * n * 2);
}

size_t trinv_ws(int64_t n) {
  Arena a(nullptr, 0);
  float* tmp;
  bf16_t* zt;
  SplitScratch sp;
  plan_trinv(a, n, &tmp, &zt, &sp);
  return a.used;
}

// Z = R^{-1} for upper-triangular R (n x n): diagonal 128-blocks (two 64
// blocks and their coupling, in LDS), then block doubling,
// Z12 = -Z11 (R12 Z22).  With ut, R holds a reflector Gram matrix G and the
// inverted matrix is its UT transform striu(G) + diag(1 + diag G) / 2 (whose
// off-diagonal blocks are G's).  fp32 levels up to 256 wide run on the
// 64-tile kernel, the rest on the GEMM engine.
static int trinv_core(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z,
                      int64_t ldz, int math, int safe, float* tmp, SplitScratch sp, bool ut,
                      int64_t w_stop) {
  const size_t esz = rdt == DT_F32 ? 4 : 2;
  const char* Rc = (const char*)R;
  if (ut && rdt != DT_F32) {
    set_error("tri_inverse: the UT transform takes an fp32 Gram matrix");
    return IFK_ERR_INVALID;
  }
  // every block on and above the diagonal is written below
  RC(launch_zero_tri_blocks(s, Z, 4, ldz, n, true));
  RC(launch_trinv_diag128(s, R, rdt, ldr, n, Z, ldz, safe, ut ? 1 : 0));
  for (int64_t w = 2 * TRINV_NB; w < n && w < w_stop; w *= 2) {
    const int64_t step = 2 * w;
    const int64_t nfull = n / step;
    const int64_t i0 = nfull * step;
    const int64_t w2 = (i0 + w < n) ? n - i0 - w : 0;   // ragged last pair
    if (math == MATH_F32 && rdt == DT_F32 && nfull + (w2 > 0 ? 1 : 0) <= SQ_BATCH) {
      // fp32: every pair of the level in one launch per product on the
      // small-product kernel: T = R12 Z22, then Z12 = -Z11 T
      const float* Rf = (const float*)R;
      SqmmArgs t1[SQ_BATCH], t2[SQ_BATCH];
      int cnt = 0;
      for (int64_t b = 0; b <= nfull; ++b) {
        const int64_t r0 = b * step, nw = b < nfull ? w : w2;
        if (nw <= 0) continue;
        float* T = tmp + (size_t)b * w * w;
        SqmmArgs x;
        x.M = w, x.N = nw, x.K = nw;
        x.A = Rf + r0 * ldr + r0 + w, x.lda = ldr;
        x.B = Z + (r0 + w) * ldz + r0 + w, x.ldb = ldz, x.trib = TRI_UPPER;
        x.out = T, x.ldo = nw;
        t1[cnt] = x;
        SqmmArgs y;
        y.M = w, y.N = nw, y.K = w;
        y.A = Z + r0 * ldz + r0, y.lda = ldz, y.tria = TRI_UPPER;
        y.B = T, y.ldb = nw;
        y.alpha = -1.0f;
        y.out = Z + r0 * ldz + r0 + w, y.ldo = ldz;
        t2[cnt] = y;
        ++cnt;
      }
      RC(launch_sqmm(s, t1, cnt));
      RC(launch_sqmm(s, t2, cnt));
      continue;
    }
    const bool small = math == MATH_F32 && rdt == DT_F32 && w <= 256;
    if (nfull > 0) {
      const void* R12 = Rc + (size_t)w * esz;  // block (0, w)
      if (small) {
        RC(launch_gemm64(s, w, w, w, 1.0f, (const float*)R12, ldr, step * (ldr + 1), TRI_NONE,
                         Z + w * ldz + w, ldz, step * (ldz + 1), TRI_UPPER, tmp, w, w * w,
                         (int)nfull));
        RC(launch_gemm64(s, w, w, w, -1.0f, Z, ldz, step * (ldz + 1), TRI_UPPER, tmp, w, w * w,
                         TRI_NONE, Z + w, ldz, step * (ldz + 1), (int)nfull));
      } else {
        RC(gemm(s, math, w, w, w, 1.0f, A_n(R12, rdt, ldr, TRI_NONE, step * (ldr + 1)),
                B_n(Z + w * ldz + w, DT_F32, ldz, TRI_UPPER, step * (ldz + 1)), 0.0f,
                out_f32(tmp, w, w * w), (int)nfull, sp));
        RC(gemm(s, math, w, w, w, -1.0f, A_n(Z, DT_F32, ldz, TRI_UPPER, step * (ldz + 1)),
                B_n(tmp, DT_F32, w, TRI_NONE, w * w), 0.0f, out_f32(Z + w, ldz, step * (ldz + 1)),
                (int)nfull, sp));
      }
    }
    if (w2 > 0) {
      // ragged pair: R12 is w x w2 and Z22 w2 x w2, so T = R12 Z22 sums over
      // w2 terms (Z22's rows end at row n - 1; a longer K would read past it)
      const void* R12 = Rc + ((size_t)i0 * ldr + i0 + w) * esz;
      if (small) {
        RC(launch_gemm64(s, w, w2, w2, 1.0f, (const float*)R12, ldr, 0, TRI_NONE,
                         Z + (i0 + w) * ldz + i0 + w, ldz, 0, TRI_UPPER, tmp, w2, 0, 1));
        RC(launch_gemm64(s, w, w2, w, -1.0f, Z + i0 * ldz + i0, ldz, 0, TRI_UPPER, tmp, w2, 0,
                         TRI_NONE, Z + i0 * ldz + i0 + w, ldz, 0, 1));
      } else {
        RC(gemm(s, math, w, w2, w2, 1.0f, A_n(R12, rdt, ldr),
                B_n(Z + (i0 + w) * ldz + i0 + w, DT_F32, ldz, TRI_UPPER), 0.0f, out_f32(tmp, w2),
                1, sp));
        RC(gemm(s, math, w, w2, w, -1.0f, A_n(Z + i0 * ldz + i0, DT_F32, ldz, TRI_UPPER),
                B_n(tmp, DT_F32, w2), 0.0f, out_f32(Z + i0 * ldz + i0 + w, ldz), 1, sp));
      }
    }
  }
  return IFK_OK;
}

// bf16-arithmetic triangular inverse that keeps two bf16 copies of Z (n x n,
// row stride ldb each): ZT = Z^T and Zb = Z, so every product reads
// K-contiguous bf16 operands: per doubling level, for the diagonal pair
// (Z11, Z22) and the block R12,
//   TmpT = ZT22 R12^T,   Z12 = -Zb11 TmpT^T (into Z and Zb),   ZT21 = Z12^T.
// tmpT: n^2 / 2 + 4 * 64^2 bf16 elements.  The products read Zb as upper
// triangular only, so its strict lower part is zeroed only on request
// (zero_zb, when Zb is handed back to the caller).
static int trinv_core_t(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z,
                        int64_t ldz, int safe, bf16_t* ZT, bf16_t* Zb, int64_t ldb, bool zero_zb,
                        bf16_t* tmpT, SplitScratch sp) {
  const int64_t NB = TRINV_NB;
  const int64_t n_ = ldb;   // row stride of both bf16 copies
  // every block on and above the diagonal of Z and Zb, and on and below it
  // of ZT, is written below: only the other triangle is cleared
  RC(launch_zero_tri_blocks(s, Z, 4, ldz, n, true));
  RC(launch_zero_tri_blocks(s, ZT, 2, n_, n, false));
  if (zero_zb) RC(launch_zero_tri_blocks(s, Zb, 2, n_, n, true));
  RC(launch_trinv_diag(s, R, rdt, ldr, n, NB, Z, ldz, safe, Zb, ZT, n_));
  return trinv_levels_t(s, R, rdt, ldr, n, NB, Z, ldz, ZT, Zb, ldb, tmpT, sp);
}

int trinv_levels_t(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, int64_t w0,
                   float* Z, int64_t ldz, bf16_t* ZT, bf16_t* Zb, int64_t ldb, bf16_t* tmpT,
                   SplitScratch sp) {
  const size_t esz = rdt == DT_F32 ? 4 : 2;
  const char* Rc = (const char*)R;
  const int64_t n_ = ldb;   // row stride of both bf16 copies
  for (int64_t w = w0; w < n; w *= 2) {
    const int64_t step = 2 * w;
    const int64_t nfull = n / step;
    if (nfull > 0) {
      const void* R12 = Rc + (size_t)w * esz;  // block (0, w) of pair 0
      RC(gemm(s, MATH_BF16, w, w, w, 1.0f, A_n(ZT + w * n_ + w, DT_BF16, n_, TRI_LOWER, step * (n_ + 1)),
              B_t(R12, rdt, ldr, TRI_NONE, step * (ldr + 1)), 0.0f, out_bf16(tmpT, w, w * w),
              (int)nfull, sp));
      RC(gemm(s, MATH_BF16, w, w, w, -1.0f, A_n(Zb, DT_BF16, n_, TRI_UPPER, step * (n_ + 1)),
              B_t(tmpT, DT_BF16, w, TRI_NONE, w * w), 0.0f,
              out_both(Z + w, ldz, Zb + w, n_, step * (ldz + 1), step * (n_ + 1)), (int)nfull, sp));
      RC(launch_transpose_cast(s, Z + w, ldz, w, w, ZT + w * n_, DT_BF16, n_, (int)nfull,
                               step * (ldz + 1), step * (n_ + 1)));
    }
    const int64_t i0 = nfull * step;
    if (i0 + w < n) {
      const int64_t w2 = n - i0 - w;
      const void* R12 = Rc + ((size_t)i0 * ldr + i0 + w) * esz;  // w x w2
      RC(gemm(s, MATH_BF16, w2, w, w2, 1.0f,
              A_n(ZT + (i0 + w) * n_ + i0 + w, DT_BF16, n_, TRI_LOWER), B_t(R12, rdt, ldr), 0.0f,
              out_bf16(tmpT, w), 1, sp));
      RC(gemm(s, MATH_BF16, w, w2, w, -1.0f, A_n(Zb + i0 * n_ + i0, DT_BF16, n_, TRI_UPPER),
              B_t(tmpT, DT_BF16, w), 0.0f,
              out_both(Z + i0 * ldz + i0 + w, ldz, Zb + i0 * n_ + i0 + w, n_), 1, sp));
      RC(launch_transpose_cast(s, Z + i0 * ldz + i0 + w, ldz, w, w2, ZT + (i0 + w) * n_ + i0,
                               DT_BF16, n_));
    }
  }
  return IFK_OK;
}

int trinv(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z, int64_t ldz,
          int math, int safe, void* ws, size_t ws_bytes) {
  if (n < 1 || ldr < n || ldz < n || !R || !Z || (rdt != DT_F32 && rdt != DT_BF16)) {
    set_error("tri_inverse: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float* tmp;
  bf16_t* zt;
  SplitScratch sp;
  plan_trinv(a, n, &tmp, &zt, &sp);
  RC(check_ws(a, "tri_inverse"));
  if (math == MATH_BF16)
    return trinv_core_t(s, R, rdt, ldr, n, Z, ldz, safe, zt, zt + (size_t)n * n, n, false,
                        (bf16_t*)tmp, sp);
  return trinv_core(s, R, rdt, ldr, n, Z, ldz, math, safe, tmp, sp);
}

// Z = R^{-1} (R upper triangular, fp32 or bf16) at about fp32 accuracy on
// bf16 MFMA.  The 128-blocks and the doubling levels up to X3_W0 / 2 wide run
// in fp32 arithmetic as in trinv_core (in LDS and on the small-product
// kernels, which are quick at those sizes); the wider levels, where the fp32
// GEMMs would cost the most, multiply split bf16 halves x = x_hi + x_lo (both
// RNE bf16) as a_hi b_hi + a_hi b_lo + a_lo b_hi (the lo.lo term dropped,
// about 2^-17 of |a||b| per product; a bf16 R has no lo half, so its products
// take two terms).  The halves of Z are kept in both layouts next to it (Zh,
// Zl row-major; ZTh, ZTl transposed, row stride n) so every product reads
// K-contiguous operands: per pair (Z11, Z22, R12) of a level
//   TmpT = ZT22 R12^T,   Z12 = -Z11 TmpT^T,
// and each new block's halves go into both copies for the wider levels.
static constexpr int64_t X3_W0 = 512;   // the first level on split bf16

struct TrinvX3Ws {
  float* tmp;
  SplitScratch sp;
  bf16_t *Zh, *Zl, *ZTh, *ZTl;   // n x n each
  bf16_t *Rh, *Rl;               // fp32 R's halves (n x n), or null
  float* T;                      // a level's TmpT blocks: n^2 / 2
  bf16_t *Th, *Tl;
};

static void plan_trinv_x3(Arena& a, int64_t n, int rdt, TrinvX3Ws& x) {
  plan_trinv(a, n, &x.tmp, &x.sp);
  const size_t nn = (size_t)n * n;
  x.Zh = a.take<bf16_t>(nn);
  x.Zl = a.take<bf16_t>(nn);
  x.ZTh = a.take<bf16_t>(nn);
  x.ZTl = a.take<bf16_t>(nn);
  x.Rh = rdt == DT_F32 ? a.take<bf16_t>(nn) : nullptr;
  x.Rl = rdt == DT_F32 ? a.take<bf16_t>(nn) : nullptr;
  x.T = a.take<float>(nn / 2 + 64);
  x.Th = a.take<bf16_t>(nn / 2 + 64);
  x.Tl = a.take<bf16_t>(nn / 2 + 64);
}

size_t trinv_x3_ws(int64_t n, int rdt) {
  Arena a(nullptr, 0);
  TrinvX3Ws x;
  plan_trinv_x3(a, n, rdt, x);
  return a.used;
}

// C (= or +=) alpha A B^T from split operands: the terms (hi, hi), (hi, lo),
// (lo, hi), each a null operand half skipped
static int gemm_split(hipStream_t s, int64_t M, int64_t N, int64_t K, float alpha,
                      const MatRef& Ah, const MatRef* Al, const MatRef& Bh, const MatRef* Bl,
                      const OutRef& out, int batch, SplitScratch sp) {
  RC(gemm(s, MATH_BF16, M, N, K, alpha, Ah, Bh, 0.0f, out, batch, sp));
  if (Bl) RC(gemm(s, MATH_BF16, M, N, K, alpha, Ah, *Bl, 1.0f, out, batch, sp));
  if (Al) RC(gemm(s, MATH_BF16, M, N, K, alpha, *Al, Bh, 1.0f, out, batch, sp));
  return IFK_OK;
}

int trinv_x3(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z, int64_t ldz,
             void* ws, size_t ws_bytes) {
  if (n < 1 || ldr < n || ldz < n || !R || !Z || (rdt != DT_F32 && rdt != DT_BF16)) {
    set_error("tri_inverse_x3: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  TrinvX3Ws x;
  plan_trinv_x3(a, n, rdt, x);
  RC(check_ws(a, "tri_inverse_x3"));
  RC(trinv_core(s, R, rdt, ldr, n, Z, ldz, MATH_F32, 0, x.tmp, x.sp, false, X3_W0));
  if (X3_W0 >= n) return IFK_OK;
  const int B16 = DT_BF16;
  // the halves of Z (its diagonal X3_W0-blocks are final; the rest is
  // written level by level below) and of an fp32 R
  RC(launch_split_bf16(s, Z, ldz, n, n, x.Zh, x.Zl, n, false));
  RC(launch_split_transpose(s, Z, ldz, n, n, x.ZTh, x.ZTl, n));
  if (rdt == DT_F32) RC(launch_split_bf16(s, (const float*)R, ldr, n, n, x.Rh, x.Rl, n, false));
  const bf16_t* Rb = rdt == DT_F32 ? x.Rh : (const bf16_t*)R;
  const int64_t ldrb = rdt == DT_F32 ? n : ldr;
  for (int64_t w = X3_W0; w < n; w *= 2) {
    const int64_t step = 2 * w;
    const int64_t nfull = n / step;
    if (nfull > 0) {
      const int64_t sa = step * (n + 1), sr = step * (ldrb + 1), sz = step * (ldz + 1);
      // TmpT = ZT22 R12^T for every full pair, batched
      const MatRef Rh12 = B_t(Rb + w, B16, ldrb, TRI_NONE, sr);
      const MatRef Rl12 = B_t(x.Rl ? x.Rl + w : nullptr, B16, ldrb, TRI_NONE, sr);
      const MatRef ZTh22 = A_n(x.ZTh + w * n + w, B16, n, TRI_LOWER, sa);
      const MatRef ZTl22 = A_n(x.ZTl + w * n + w, B16, n, TRI_LOWER, sa);
      RC(gemm_split(s, w, w, w, 1.0f, ZTh22, &ZTl22, Rh12, x.Rl ? &Rl12 : nullptr,
                    out_f32(x.T, w, w * w), (int)nfull, x.sp));
      RC(launch_split_bf16(s, x.T, w, nfull * w, w, x.Th, x.Tl, w, false));
      // Z12 = -Z11 TmpT^T
      const MatRef Zh11 = A_n(x.Zh, B16, n, TRI_UPPER, sa), Zl11 = A_n(x.Zl, B16, n, TRI_UPPER, sa);
      const MatRef Th = B_t(x.Th, B16, w, TRI_NONE, w * w), Tl = B_t(x.Tl, B16, w, TRI_NONE, w * w);
      RC(gemm_split(s, w, w, w, -1.0f, Zh11, &Zl11, Th, &Tl, out_f32(Z + w, ldz, sz), (int)nfull,
                    x.sp));
      for (int64_t b = 0; b < nfull; ++b) {
        const int64_t r0 = b * step;
        const float* Z12 = Z + r0 * ldz + r0 + w;
        RC(launch_split_bf16(s, Z12, ldz, w, w, x.Zh + r0 * n + r0 + w, x.Zl + r0 * n + r0 + w, n,
                             false));
        RC(launch_split_transpose(s, Z12, ldz, w, w, x.ZTh + (r0 + w) * n + r0,
                                  x.ZTl + (r0 + w) * n + r0, n));
      }
    }
    const int64_t i0 = nfull * step;
    if (i0 + w < n) {
      const int64_t w2 = n - i0 - w;   // ragged pair: Z22 is w2 x w2, R12 w x w2
      const MatRef Rh12 = B_t(Rb + i0 * ldrb + i0 + w, B16, ldrb);
      const MatRef Rl12 = B_t(x.Rl ? x.Rl + i0 * ldrb + i0 + w : nullptr, B16, ldrb);
      const MatRef ZTh22 = A_n(x.ZTh + (i0 + w) * n + i0 + w, B16, n, TRI_LOWER);
      const MatRef ZTl22 = A_n(x.ZTl + (i0 + w) * n + i0 + w, B16, n, TRI_LOWER);
      RC(gemm_split(s, w2, w, w2, 1.0f, ZTh22, &ZTl22, Rh12, x.Rl ? &Rl12 : nullptr,
                    out_f32(x.T, w), 1, x.sp));
      RC(launch_split_bf16(s, x.T, w, w2, w, x.Th, x.Tl, w, false));
      const MatRef Zh11 = A_n(x.Zh + i0 * n + i0, B16, n, TRI_UPPER);
      const MatRef Zl11 = A_n(x.Zl + i0 * n + i0, B16, n, TRI_UPPER);
      const MatRef Th = B_t(x.Th, B16, w), Tl = B_t(x.Tl, B16, w);
      float* Z12 = Z + i0 * ldz + i0 + w;
      RC(gemm_split(s, w, w2, w, -1.0f, Zh11, &Zl11, Th, &Tl, out_f32(Z12, ldz), 1, x.sp));
      RC(launch_split_bf16(s, Z12, ldz, w, w2, x.Zh + i0 * n + i0 + w, x.Zl + i0 * n + i0 + w, n,
                           false));
      RC(launch_split_transpose(s, Z12, ldz, w, w2, x.ZTh + (i0 + w) * n + i0,
                                x.ZTl + (i0 + w) * n + i0, n));
    }
  }
  return IFK_OK;
}

int trinv_copies(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z,
                 int64_t ldz, bf16_t* Zb, bf16_t* ZTb, int64_t ldb, void* ws, size_t ws_bytes) {
  if (n < 1 || ldr < n || ldz < n || ldb < n || !R || !Z || !Zb || !ZTb ||
      (rdt != DT_F32 && rdt != DT_BF16)) {
    set_error("tri_inverse_bf16: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float* tmp;
  SplitScratch sp;
  plan_trinv(a, n, &tmp, &sp);
  RC(check_ws(a, "tri_inverse_bf16"));
  return trinv_core_t(s, R, rdt, ldr, n, Z, ldz, 0, ZTb, Zb, ldb, true, (bf16_t*)tmp, sp);
}

size_t trinv_copies_ws(int64_t n) {
  Arena a(nullptr, 0);
  float* tmp;
  SplitScratch sp;
  plan_trinv(a, n, &tmp, &sp);
  return a.used;
}

// ----------------------------------------------------------------------------
// Condition estimate
// ----------------------------------------------------------------------------
// kappa_2(R) ~ sigma_max(R) sigma_max(Z) for an upper-triangular R and its
// inverse Z, each sigma_max by COND_IT steps of block power iteration
// (v <- M^T M v, COND_K probe vectors) on the fp32 GEMM engine.  The power
// iteration approaches sigma_max from below, so the estimate is a lower
// bound: within a few percent after four steps when the extreme singular
// values are spread, within about 10 % when they cluster (the smallest ones
// of a factor whose input has a dominant mean direction).
static constexpr int COND_K = 4;
static constexpr int COND_IT = 4;

static void plan_cond(Arena& a, int64_t n, float** V, float** W, float** ss, SplitScratch* sp) {
  *V = a.take<float>((size_t)n * COND_K);
  *W = a.take<float>((size_t)n * COND_K);
  *ss = a.take<float>(2 * COND_K);
  sp->floats = (size_t)64 * n * COND_K;
  sp->p = a.take<float>(sp->floats);
}

size_t cond_est_ws(int64_t n) {
  Arena a(nullptr, 0);
  float *V, *W, *ss;
  SplitScratch sp;
  plan_cond(a, n, &V, &W, &ss, &sp);
  return a.used;
}

int cond_est(hipStream_t s, const void* R, int rdt, int64_t ldr, const float* Z, int64_t ldz,
             int64_t n, float* kappa, void* ws, size_t ws_bytes) {
  if (n < 1 || ldr < n || ldz < n || !R || !Z || !kappa || (rdt != DT_F32 && rdt != DT_BF16)) {
    set_error("cond_estimate: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float *V, *W, *ss;
  SplitScratch sp;
  plan_cond(a, n, &V, &W, &ss, &sp);
  RC(check_ws(a, "cond_estimate"));
  for (int m = 0; m < 2; ++m) {
    const void* M = m == 0 ? R : (const void*)Z;
    const int dt = m == 0 ? rdt : DT_F32;
    const int64_t ld = m == 0 ? ldr : ldz;
    RC(launch_probe_init(s, V, n, COND_K));
    RC(launch_colnorm(s, V, n, COND_K, ss + m * COND_K));
    for (int it = 0; it < COND_IT; ++it) {
      RC(gemm(s, MATH_F32, n, COND_K, n, 1.0f, A_n(M, dt, ld, TRI_UPPER), B_n(V, DT_F32, COND_K),
              0.0f, out_f32(W, COND_K), 1, sp));
      RC(gemm(s, MATH_F32, n, COND_K, n, 1.0f, A_t(M, dt, ld, TRI_LOWER), B_n(W, DT_F32, COND_K),
              0.0f, out_f32(V, COND_K), 1, sp));
      RC(launch_colnorm(s, V, n, COND_K, ss + m * COND_K));
    }
  }
  return launch_cond_final(s, ss, ss + COND_K, COND_K, kappa);
}

// ----------------------------------------------------------------------------
// Preconditioning
// ----------------------------------------------------------------------------
static void plan_apply(Arena& a, int64_t n_out, int64_t n_in, int math, void** T1, void** T2,
                       bf16_t** cv, SplitScratch* sp) {
  const size_t e = (size_t)n_out * n_in;
  *cv = nullptr;
  if (math == MATH_BF16) {
    *T1 = a.take<bf16_t>(e);
    *T2 = a.take<bf16_t>(e);
    *cv = a.take<bf16_t>(e + 2 * (size_t)n_out * n_out + 2 * (size_t)n_in * n_in);
  } else {
    *T1 = a.take<float>(e);
    *T2 = a.take<float>(e);
  }
  sp->floats = split_floats(TRINV_NB, std::max(n_out, n_in));
  sp->p = a.take<float>(sp->floats);
}

// ... for precondition_apply_b: only grad^T is cast.  The split-K scratch
// holds at most split_cap floats (the GEMM engine uses fewer splits when it
// is smaller, never failing for lack of it).
static void plan_apply_b(Arena& a, int64_t n_out, int64_t n_in, void** T1, void** T2,
                         bf16_t** cv, SplitScratch* sp, size_t split_cap = SIZE_MAX) {
  const size_t e = (size_t)n_out * n_in;
  *T1 = a.take<bf16_t>(e);
  *T2 = a.take<bf16_t>(e);
  *cv = a.take<bf16_t>(e);
  sp->floats = std::min(split_floats(TRINV_NB, std::max(n_out, n_in)), split_cap);
  sp->p = a.take<float>(sp->floats);
}

size_t precondition_apply_ws(int64_t n_out, int64_t n_in, int math) {
  Arena a(nullptr, 0);
  void *T1, *T2;
  bf16_t* cv;
  SplitScratch sp;
  plan_apply(a, n_out, n_in, math, &T1, &T2, &cv, &sp);
  return a.used;
}

// The bf16 products of the apply, given bf16 copies (the RNE roundings the
// MFMA operands get anyway) of grad^T (gT, n_in x n_out), Z_G and Z_G^T (ld
// ldg2), Z_X and Z_X^T (ld ldx2): every product reads both operands
// K-contiguous.  Only the upper triangle of ZGb, ZXb and the lower triangle of
// ZGt, ZXt are read.
static int apply_core_b(hipStream_t s, const bf16_t* gT, int64_t n_out, int64_t n_in,
                        const bf16_t* ZXb, const bf16_t* ZXt, int64_t ldx2, const bf16_t* ZGb,
                        const bf16_t* ZGt, int64_t ldg2, float* nat, int64_t ldn, void* T1,
                        void* T2, SplitScratch sp) {
  const int math = MATH_BF16;
  bf16_t* T1T = (bf16_t*)T1;   // n_in x n_out
  bf16_t* Tb = (bf16_t*)T2;    // n_out x n_in
  // T1^T = grad^T Z_G          (T1 = Z_G^T grad: R_G^T T1 = grad, triangular.py:632)
  RC(gemm(s, math, n_in, n_out, n_out, 1.0f, A_n(gT, DT_BF16, n_out),
          B_t(ZGt, DT_BF16, ldg2, TRI_UPPER), 0.0f, out_bf16(T1T, n_out), 1, sp));
  // T2 = Z_G T1                (R_G T2 = T1, triangular.py:636)
  RC(gemm(s, math, n_out, n_in, n_out, 1.0f, A_n(ZGb, DT_BF16, ldg2, TRI_UPPER),
          B_t(T1T, DT_BF16, n_out), 0.0f, out_bf16(Tb, n_in), 1, sp));
  // T3 = T2 Z_X                (R_X^T T3^T = T2^T, triangular.py:645), into T1's buffer
  RC(gemm(s, math, n_out, n_in, n_in, 1.0f, A_n(Tb, DT_BF16, n_in),
          B_t(ZXt, DT_BF16, ldx2, TRI_UPPER), 0.0f, out_bf16(T1T, n_in), 1, sp));
  // nat = T3 Z_X^T             (R_X T4^T = T3^T, triangular.py:649)
  return gemm(s, math, n_out, n_in, n_in, 1.0f, A_n(T1T, DT_BF16, n_in),
              B_t(ZXb, DT_BF16, ldx2, TRI_LOWER), 0.0f, out_f32(nat, ldn), 1, sp);
}

// ----------------------------------------------------------------------------
// The apply at fp32 accuracy on bf16 MFMA: every operand x = x_hi + x_lo (RNE
// bf16 halves) and every product a b as a_hi b_hi + a_hi b_lo + a_lo b_hi --
// three launches into one fp32 result, each keeping the triangular operand's
// K trimming; the dropped lo.lo term and the roundings leave about 2^-17 of
// |a||b| per product.  This is the arithmetic for factors whose kappa makes the
// bf16 apply's rounding visible (the reference's regime, fp32 solves on the
// bf16-valued factors, triangular.py:621-628, to the same order).
// ----------------------------------------------------------------------------
int split_inverse(hipStream_t s, const float* Z, int64_t ldz, int64_t n, bf16_t* Zh, bf16_t* Zl,
                  bf16_t* ZTh, bf16_t* ZTl, int64_t ldb) {
  if (n < 1 || ldz < n || ldb < n || !Z || !Zh || !Zl || !ZTh || !ZTl) {
    set_error("inverse_split_copies: invalid arguments");
    return IFK_ERR_INVALID;
  }
  RC(launch_split_bf16(s, Z, ldz, n, n, Zh, Zl, ldb, false));
  return launch_split_transpose(s, Z, ldz, n, n, ZTh, ZTl, ldb);
}

static void plan_apply_x3(Arena& a, int64_t n_out, int64_t n_in, float** T, bf16_t** Sh,
                          bf16_t** Sl, bf16_t** gTh, bf16_t** gTl, SplitScratch* sp) {
  const size_t e = (size_t)n_out * n_in;
  *T = a.take<float>(e);
  *Sh = a.take<bf16_t>(e);
  *Sl = a.take<bf16_t>(e);
  *gTh = a.take<bf16_t>(e);
  *gTl = a.take<bf16_t>(e);
  sp->floats = split_floats(TRINV_NB, std::max(n_out, n_in));
  sp->p = a.take<float>(sp->floats);
}

size_t precondition_apply_x3_ws(int64_t n_out, int64_t n_in) {
  Arena a(nullptr, 0);
  float* T;
  bf16_t *Sh, *Sl, *gTh, *gTl;
  SplitScratch sp;
  plan_apply_x3(a, n_out, n_in, &T, &Sh, &Sl, &gTh, &gTl, &sp);
  return a.used;
}

// C (fp32, ldc) = op(A) op(B) from the halves (A_hi, A_lo) and (B_hi, B_lo)
static int gemm_x3(hipStream_t s, int64_t M, int64_t N, int64_t K, const MatRef& Ah,
                   const MatRef& Al, const MatRef& Bh, const MatRef& Bl, float* C, int64_t ldc,
                   SplitScratch sp) {
  RC(gemm(s, MATH_BF16, M, N, K, 1.0f, Ah, Bh, 0.0f, out_f32(C, ldc), 1, sp));
  RC(gemm(s, MATH_BF16, M, N, K, 1.0f, Ah, Bl, 1.0f, out_f32(C, ldc), 1, sp));
  return gemm(s, MATH_BF16, M, N, K, 1.0f, Al, Bh, 1.0f, out_f32(C, ldc), 1, sp);
}

int precondition_apply_x3(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in,
                          int64_t ldg, const bf16_t* const* ZX, int64_t ldx,
                          const bf16_t* const* ZG, int64_t ldg2, float* nat, int64_t ldn, void* ws,
                          size_t ws_bytes) {
  if (n_out < 1 || n_in < 1 || ldg < n_in || ldn < n_in || ldx < n_in || ldg2 < n_out || !grad ||
      !nat || !ZX || !ZG || !ZX[0] || !ZX[1] || !ZX[2] || !ZX[3] || !ZG[0] || !ZG[1] || !ZG[2] ||
      !ZG[3]) {
    set_error("precondition_apply_x3: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float* T;
  bf16_t *Sh, *Sl, *gTh, *gTl;
  SplitScratch sp;
  plan_apply_x3(a, n_out, n_in, &T, &Sh, &Sl, &gTh, &gTl, &sp);
  RC(check_ws(a, "precondition_apply_x3"));
  const int B16 = DT_BF16;
  // ZX / ZG: [Z_hi, Z_lo, Z^T_hi, Z^T_lo]
  RC(launch_split_transpose(s, grad, ldg, n_out, n_in, gTh, gTl, n_out));
  // T1^T = grad^T Z_G (n_in x n_out)
  RC(gemm_x3(s, n_in, n_out, n_out, A_n(gTh, B16, n_out), A_n(gTl, B16, n_out),
             B_t(ZG[2], B16, ldg2, TRI_UPPER), B_t(ZG[3], B16, ldg2, TRI_UPPER), T, n_out, sp));
  RC(launch_split_bf16(s, T, n_out, n_in, n_out, Sh, Sl, n_out, false));
  // T2 = Z_G T1 (n_out x n_in)
  RC(gemm_x3(s, n_out, n_in, n_out, A_n(ZG[0], B16, ldg2, TRI_UPPER),
             A_n(ZG[1], B16, ldg2, TRI_UPPER), B_t(Sh, B16, n_out), B_t(Sl, B16, n_out), T, n_in,
             sp));
  RC(launch_split_bf16(s, T, n_in, n_out, n_in, Sh, Sl, n_in, false));
  // T3 = T2 Z_X
  RC(gemm_x3(s, n_out, n_in, n_in, A_n(Sh, B16, n_in), A_n(Sl, B16, n_in),
             B_t(ZX[2], B16, ldx, TRI_UPPER), B_t(ZX[3], B16, ldx, TRI_UPPER), T, n_in, sp));
  RC(launch_split_bf16(s, T, n_in, n_out, n_in, Sh, Sl, n_in, false));
  // nat = T3 Z_X^T
  return gemm_x3(s, n_out, n_in, n_in, A_n(Sh, B16, n_in), A_n(Sl, B16, n_in),
                 B_t(ZX[0], B16, ldx, TRI_LOWER), B_t(ZX[1], B16, ldx, TRI_LOWER), nat, ldn, sp);
}

static int apply_core(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in, int64_t ldg,
                      const float* ZX, int64_t ldzx, const float* ZG, int64_t ldzg, float* nat,
                      int64_t ldn, int math, void* T1, void* T2, bf16_t* cv, SplitScratch sp) {
  if (math == MATH_BF16) {
    bf16_t* gT = cv;                                   // n_in x n_out
    bf16_t* ZGb = gT + (size_t)n_in * n_out;           // n_out x n_out
    bf16_t* ZGt = ZGb + (size_t)n_out * n_out;
    bf16_t* ZXb = ZGt + (size_t)n_out * n_out;         // n_in x n_in
    bf16_t* ZXt = ZXb + (size_t)n_in * n_in;
    RC(launch_transpose_cast(s, grad, ldg, n_out, n_in, gT, DT_BF16, n_out));
    RC(launch_cast(s, ZG, ldzg, n_out, n_out, ZGb, DT_BF16, n_out));
    RC(launch_transpose_cast(s, ZG, ldzg, n_out, n_out, ZGt, DT_BF16, n_out));
    RC(launch_cast(s, ZX, ldzx, n_in, n_in, ZXb, DT_BF16, n_in));
    RC(launch_transpose_cast(s, ZX, ldzx, n_in, n_in, ZXt, DT_BF16, n_in));
    return apply_core_b(s, gT, n_out, n_in, ZXb, ZXt, n_in, ZGb, ZGt, n_out, nat, ldn, T1, T2, sp);
  }
  const int tdt = DT_F32;
  auto out_t = [&](void* p, int64_t ld) {
    return tdt == DT_BF16 ? out_bf16((bf16_t*)p, ld) : out_f32((float*)p, ld);
  };
  // T1 = Z_G^T grad        (R_G^T T1 = grad, triangular.py:632)
  RC(gemm(s, math, n_out, n_in, n_out, 1.0f, A_t(ZG, DT_F32, ldzg, TRI_LOWER),
          B_n(grad, DT_F32, ldg), 0.0f, out_t(T1, n_in), 1, sp));
  // T2 = Z_G T1            (R_G T2 = T1, triangular.py:636)
  RC(gemm(s, math, n_out, n_in, n_out, 1.0f, A_n(ZG, DT_F32, ldzg, TRI_UPPER),
          B_n(T1, tdt, n_in), 0.0f, out_t(T2, n_in), 1, sp));
  // T3 = T2 Z_X            (R_X^T T3^T = T2^T, triangular.py:645)
  RC(gemm(s, math, n_out, n_in, n_in, 1.0f, A_n(T2, tdt, n_in),
          B_n(ZX, DT_F32, ldzx, TRI_UPPER), 0.0f, out_t(T1, n_in), 1, sp));
  // nat = T3 Z_X^T         (R_X T4^T = T3^T, triangular.py:649)
  RC(gemm(s, math, n_out, n_in, n_in, 1.0f, A_n(T1, tdt, n_in),
          B_t(ZX, DT_F32, ldzx, TRI_LOWER), 0.0f, out_f32(nat, ldn), 1, sp));
  return IFK_OK;
}

int precondition_apply(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in, int64_t ldg,
                       const float* ZX, int64_t ldzx, const float* ZG, int64_t ldzg, float* nat,
                       int64_t ldn, int math, void* ws, size_t ws_bytes) {
  if (n_out < 1 || n_in < 1 || ldg < n_in || ldn < n_in || ldzx < n_in || ldzg < n_out || !grad ||
      !ZX || !ZG || !nat) {
    set_error("precondition_apply: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  void *T1, *T2;
  bf16_t* cv;
  SplitScratch sp;
  plan_apply(a, n_out, n_in, math, &T1, &T2, &cv, &sp);
  RC(check_ws(a, "precondition_apply"));
  return apply_core(s, grad, n_out, n_in, ldg, ZX, ldzx, ZG, ldzg, nat, ldn, math, T1, T2, cv, sp);
}

// nat from grad and the bf16 copies written by trinv_copies
int precondition_apply_b(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in,
                         int64_t ldg, const bf16_t* ZXb, const bf16_t* ZXt, int64_t ldx2,
                         const bf16_t* ZGb, const bf16_t* ZGt, int64_t ldg2, float* nat,
                         int64_t ldn, void* ws, size_t ws_bytes) {
  if (n_out < 1 || n_in < 1 || ldg < n_in || ldn < n_in || ldx2 < n_in || ldg2 < n_out || !grad ||
      !ZXb || !ZXt || !ZGb || !ZGt || !nat) {
    set_error("precondition_apply_bf16: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  void *T1, *T2;
  bf16_t* cv;
  SplitScratch sp;
  plan_apply_b(a, n_out, n_in, &T1, &T2, &cv, &sp);
  RC(check_ws(a, "precondition_apply_bf16"));
  RC(launch_transpose_cast(s, grad, ldg, n_out, n_in, cv, DT_BF16, n_out));
  return apply_core_b(s, cv, n_out, n_in, ZXb, ZXt, ldx2, ZGb, ZGt, ldg2, nat, ldn, T1, T2, sp);
}

size_t precondition_apply_b_ws(int64_t n_out, int64_t n_in) {
  Arena a(nullptr, 0);
  void *T1, *T2;
  bf16_t* cv;
  SplitScratch sp;
  plan_apply_b(a, n_out, n_in, &T1, &T2, &cv, &sp);
  return a.used;
}

size_t precondition_apply_b_min_ws(int64_t n_out, int64_t n_in) {
  Arena a(nullptr, 0);
  void *T1, *T2;
  bf16_t* cv;
  SplitScratch sp;
  plan_apply_b(a, n_out, n_in, &T1, &T2, &cv, &sp, 0);
  return a.used;
}

// ---------------------------------------------------------------------------
// The applies for B layers of one shape (grouped launches).  Every product is
// one launch over the batch with per-entry tile and split-K choices, and the
// split-K scratch is B times a single call's, so each entry gets exactly the
// bits precondition_apply_b / precondition_apply_x3 give it alone.  The
// intermediate buffers are B-strided (E = n_out n_in elements per entry).
// ---------------------------------------------------------------------------
static void plan_apply_b_batched(Arena& a, int64_t B, int64_t n_out, int64_t n_in, bf16_t** T1,
                                 bf16_t** T2, bf16_t** cv, SplitScratch* sp) {
  const size_t e = (size_t)B * n_out * n_in;
  *T1 = a.take<bf16_t>(e);
  *T2 = a.take<bf16_t>(e);
  *cv = a.take<bf16_t>(e);
  sp->floats = (size_t)B * split_floats(TRINV_NB, std::max(n_out, n_in));
  sp->p = a.take<float>(sp->floats);
}

size_t precondition_apply_b_batched_ws(int64_t batch, int64_t n_out, int64_t n_in) {
  Arena a(nullptr, 0);
  bf16_t *T1, *T2, *cv;
  SplitScratch sp;
  plan_apply_b_batched(a, batch, n_out, n_in, &T1, &T2, &cv, &sp);
  return a.used;
}

static bool batch_args_ok(int64_t B, const float* const* grad, int64_t n_out, int64_t n_in,
                          int64_t ldg, int64_t ldn, int64_t snat, const float* nat) {
  if (B < 1 || B > 65535 || n_out < 1 || n_in < 1 || ldg < n_in || ldn < n_in || !grad || !nat ||
      (B > 1 && snat < n_out * ldn))
    return false;
  for (int64_t e = 0; e < B; ++e)
    if (!grad[e]) return false;
  return true;
}

int precondition_apply_b_batched(hipStream_t s, int64_t B, const float* const* grad,
                                 int64_t n_out, int64_t n_in, int64_t ldg, const bf16_t* ZXb,
                                 const bf16_t* ZXt, int64_t ldx2, int64_t sx, const bf16_t* ZGb,
                                 const bf16_t* ZGt, int64_t ldg2, int64_t sg, float* nat,
                                 int64_t ldn, int64_t snat, void* ws, size_t ws_bytes) {
  if (!batch_args_ok(B, grad, n_out, n_in, ldg, ldn, snat, nat) || ldx2 < n_in ||
      ldg2 < n_out || !ZXb || !ZXt || !ZGb || !ZGt ||
      (B > 1 && (sx < n_in * ldx2 || sg < n_out * ldg2))) {
    set_error("precondition_apply_bf16_batched: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  bf16_t *T1T, *Tb, *cv;
  SplitScratch sp;
  plan_apply_b_batched(a, B, n_out, n_in, &T1T, &Tb, &cv, &sp);
  RC(check_ws(a, "precondition_apply_bf16_batched"));
  const int64_t E = n_out * n_in;
  const int math = MATH_BF16, nb = (int)B;
  for (int64_t e = 0; e < B; ++e)
    RC(launch_transpose_cast(s, grad[e], ldg, n_out, n_in, cv + e * E, DT_BF16, n_out));
  // the four products of apply_core_b, each over the batch
  RC(gemm(s, math, n_in, n_out, n_out, 1.0f, A_n(cv, DT_BF16, n_out, TRI_NONE, E),
          B_t(ZGt, DT_BF16, ldg2, TRI_UPPER, sg), 0.0f, per_entry(out_bf16(T1T, n_out, E)), nb,
          sp));
  RC(gemm(s, math, n_out, n_in, n_out, 1.0f, A_n(ZGb, DT_BF16, ldg2, TRI_UPPER, sg),
          B_t(T1T, DT_BF16, n_out, TRI_NONE, E), 0.0f, per_entry(out_bf16(Tb, n_in, E)), nb, sp));
  RC(gemm(s, math, n_out, n_in, n_in, 1.0f, A_n(Tb, DT_BF16, n_in, TRI_NONE, E),
          B_t(ZXt, DT_BF16, ldx2, TRI_UPPER, sx), 0.0f, per_entry(out_bf16(T1T, n_in, E)), nb,
          sp));
  return gemm(s, math, n_out, n_in, n_in, 1.0f, A_n(T1T, DT_BF16, n_in, TRI_NONE, E),
              B_t(ZXb, DT_BF16, ldx2, TRI_LOWER, sx), 0.0f, per_entry(out_f32(nat, ldn, snat)),
              nb, sp);
}

static void plan_apply_x3_batched(Arena& a, int64_t B, int64_t n_out, int64_t n_in, float** T,
                                  bf16_t** Sh, bf16_t** Sl, bf16_t** gTh, bf16_t** gTl,
                                  SplitScratch* sp) {
  const size_t e = (size_t)B * n_out * n_in;
  *T = a.take<float>(e);
  *Sh = a.take<bf16_t>(e);
  *Sl = a.take<bf16_t>(e);
  *gTh = a.take<bf16_t>(e);
  *gTl = a.take<bf16_t>(e);
  sp->floats = (size_t)B * split_floats(TRINV_NB, std::max(n_out, n_in));
  sp->p = a.take<float>(sp->floats);
}

size_t precondition_apply_x3_batched_ws(int64_t batch, int64_t n_out, int64_t n_in) {
  Arena a(nullptr, 0);
  float* T;
  bf16_t *Sh, *Sl, *gTh, *gTl;
  SplitScratch sp;
  plan_apply_x3_batched(a, batch, n_out, n_in, &T, &Sh, &Sl, &gTh, &gTl, &sp);
  return a.used;
}

// C (fp32, ldc, entry stride sc) = op(A) op(B) from the halves, B entries
static int gemm_x3_batched(hipStream_t s, int B, int64_t M, int64_t N, int64_t K,
                           const MatRef& Ah, const MatRef& Al, const MatRef& Bh,
                           const MatRef& Bl, float* C, int64_t ldc, int64_t sc, SplitScratch sp) {
  RC(gemm(s, MATH_BF16, M, N, K, 1.0f, Ah, Bh, 0.0f, per_entry(out_f32(C, ldc, sc)), B, sp));
  RC(gemm(s, MATH_BF16, M, N, K, 1.0f, Ah, Bl, 1.0f, per_entry(out_f32(C, ldc, sc)), B, sp));
  return gemm(s, MATH_BF16, M, N, K, 1.0f, Al, Bh, 1.0f, per_entry(out_f32(C, ldc, sc)), B, sp);
}

int precondition_apply_x3_batched(hipStream_t s, int64_t B, const float* const* grad,
                                  int64_t n_out, int64_t n_in, int64_t ldg,
                                  const bf16_t* const* ZX, int64_t ldx, int64_t sx,
                                  const bf16_t* const* ZG, int64_t ldg2, int64_t sg, float* nat,
                                  int64_t ldn, int64_t snat, void* ws, size_t ws_bytes) {
  bool ok = batch_args_ok(B, grad, n_out, n_in, ldg, ldn, snat, nat) && ldx >= n_in &&
            ldg2 >= n_out && ZX && ZG && (B == 1 || (sx >= n_in * ldx && sg >= n_out * ldg2));
  for (int i = 0; ok && i < 4; ++i) ok = ZX[i] && ZG[i];
  if (!ok) {
    set_error("precondition_apply_x3_batched: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float* T;
  bf16_t *Sh, *Sl, *gTh, *gTl;
  SplitScratch sp;
  plan_apply_x3_batched(a, B, n_out, n_in, &T, &Sh, &Sl, &gTh, &gTl, &sp);
  RC(check_ws(a, "precondition_apply_x3_batched"));
  const int B16 = DT_BF16, nb = (int)B;
  const int64_t E = n_out * n_in;
  for (int64_t e = 0; e < B; ++e)
    RC(launch_split_transpose(s, grad[e], ldg, n_out, n_in, gTh + e * E, gTl + e * E, n_out));
  // T1^T = grad^T Z_G (n_in x n_out per entry)
  RC(gemm_x3_batched(s, nb, n_in, n_out, n_out, A_n(gTh, B16, n_out, TRI_NONE, E),
                     A_n(gTl, B16, n_out, TRI_NONE, E), B_t(ZG[2], B16, ldg2, TRI_UPPER, sg),
                     B_t(ZG[3], B16, ldg2, TRI_UPPER, sg), T, n_out, E, sp));
  // the batch's entries are consecutive rows of the same width: one split each
  RC(launch_split_bf16(s, T, n_out, B * n_in, n_out, Sh, Sl, n_out, false));
  // T2 = Z_G T1 (n_out x n_in)
  RC(gemm_x3_batched(s, nb, n_out, n_in, n_out, A_n(ZG[0], B16, ldg2, TRI_UPPER, sg),
                     A_n(ZG[1], B16, ldg2, TRI_UPPER, sg), B_t(Sh, B16, n_out, TRI_NONE, E),
                     B_t(Sl, B16, n_out, TRI_NONE, E), T, n_in, E, sp));
  RC(launch_split_bf16(s, T, n_in, B * n_out, n_in, Sh, Sl, n_in, false));
  // T3 = T2 Z_X
  RC(gemm_x3_batched(s, nb, n_out, n_in, n_in, A_n(Sh, B16, n_in, TRI_NONE, E),
                     A_n(Sl, B16, n_in, TRI_NONE, E), B_t(ZX[2], B16, ldx, TRI_UPPER, sx),
                     B_t(ZX[3], B16, ldx, TRI_UPPER, sx), T, n_in, E, sp));
  RC(launch_split_bf16(s, T, n_in, B * n_out, n_in, Sh, Sl, n_in, false));
  // nat = T3 Z_X^T
  return gemm_x3_batched(s, nb, n_out, n_in, n_in, A_n(Sh, B16, n_in, TRI_NONE, E),
                         A_n(Sl, B16, n_in, TRI_NONE, E), B_t(ZX[0], B16, ldx, TRI_LOWER, sx),
                         B_t(ZX[1], B16, ldx, TRI_LOWER, sx), nat, ldn, snat, sp);
}

// precondition_apply_b in a workspace of any size from
// precondition_apply_b_min_ws up: the split-K scratch gets what is left after
// the operand buffers, up to what precondition_apply_b would take (with that
// much room the two run the same launches and give the same bits).
int precondition_apply_b_fit(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in,
                             int64_t ldg, const bf16_t* ZXb, const bf16_t* ZXt, int64_t ldx2,
                             const bf16_t* ZGb, const bf16_t* ZGt, int64_t ldg2, float* nat,
                             int64_t ldn, void* ws, size_t ws_bytes) {
  if (n_out < 1 || n_in < 1 || ldg < n_in || ldn < n_in || ldx2 < n_in || ldg2 < n_out || !grad ||
      !ZXb || !ZXt || !ZGb || !ZGt || !nat) {
    set_error("precondition_apply_bf16: invalid arguments");
    return IFK_ERR_INVALID;
  }
  const size_t need = precondition_apply_b_min_ws(n_out, n_in);
  const size_t room = ws_bytes > need + 256 ? (ws_bytes - need - 256) / sizeof(float) : 0;
  Arena a(ws, ws_bytes);
  void *T1, *T2;
  bf16_t* cv;
  SplitScratch sp;
  plan_apply_b(a, n_out, n_in, &T1, &T2, &cv, &sp, room);
  RC(check_ws(a, "precondition_apply_bf16"));
  RC(launch_transpose_cast(s, grad, ldg, n_out, n_in, cv, DT_BF16, n_out));
  return apply_core_b(s, cv, n_out, n_in, ZXb, ZXt, ldx2, ZGb, ZGt, ldg2, nat, ldn, T1, T2, sp);
}

static void plan_prec(Arena& a, int64_t n_out, int64_t n_in, int math, float** ZX, float** ZG,
                      float** tmp, bf16_t** zt, SplitScratch* tsp, void** T1, void** T2,
                      bf16_t** cv, SplitScratch* asp) {
  *ZX = a.take<float>((size_t)n_in * n_in);
  *ZG = a.take<float>((size_t)n_out * n_out);
  plan_trinv(a, std::max(n_in, n_out), tmp, zt, tsp);
  plan_apply(a, n_out, n_in, math, T1, T2, cv, asp);
}

size_t precondition_ws(int64_t n_out, int64_t n_in, int math) {
  Arena a(nullptr, 0);
  float *ZX, *ZG, *tmp;
  bf16_t *zt, *cv;
  void *T1, *T2;
  SplitScratch tsp, asp;
  plan_prec(a, n_out, n_in, math, &ZX, &ZG, &tmp, &zt, &tsp, &T1, &T2, &cv, &asp);
  return a.used;
}

int precondition(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in, int64_t ldg,
                 const void* RX, int64_t ldrx, const void* RG, int64_t ldrg, int rdt, float* nat,
                 int64_t ldn, int math, void* ws, size_t ws_bytes) {
  if (n_out < 1 || n_in < 1 || ldg < n_in || ldn < n_in || ldrx < n_in || ldrg < n_out || !grad ||
      !RX || !RG || !nat || (rdt != DT_F32 && rdt != DT_BF16)) {
    set_error("precondition: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float *ZX, *ZG, *tmp;
  bf16_t *zt, *cv;
  void *T1, *T2;
  SplitScratch tsp, asp;
  plan_prec(a, n_out, n_in, math, &ZX, &ZG, &tmp, &zt, &tsp, &T1, &T2, &cv, &asp);
  RC(check_ws(a, "precondition"));
  if (math == MATH_BF16) {
    RC(trinv_core_t(s, RX, rdt, ldrx, n_in, ZX, n_in, 0, zt, zt + (size_t)n_in * n_in, n_in, false,
                    (bf16_t*)tmp, tsp));
    RC(trinv_core_t(s, RG, rdt, ldrg, n_out, ZG, n_out, 0, zt, zt + (size_t)n_out * n_out, n_out,
                    false, (bf16_t*)tmp, tsp));
  } else {
    RC(trinv_core(s, RX, rdt, ldrx, n_in, ZX, n_in, math, 0, tmp, tsp));
    RC(trinv_core(s, RG, rdt, ldrg, n_out, ZG, n_out, math, 0, tmp, tsp));
  }
  return apply_core(s, grad, n_out, n_in, ldg, ZX, n_in, ZG, n_out, nat, ldn, math, T1, T2, cv,
                    asp);
}

size_t precondition_bias_ws(int64_t n_out) {
  Arena a(nullptr, 0);
  a.take<float>(n_out);
  SplitScratch sp;
  sp.floats = split_floats(TRINV_NB, n_out);
  a.take<float>(sp.floats);
  return a.used;
}

int precondition_bias(hipStream_t s, const float* g, int64_t n_out, const float* ZG, int64_t ldzg,
                      float* out, void* ws, size_t ws_bytes) {
  if (n_out < 1 || ldzg < n_out || !g || !ZG || !out) {
    set_error("precondition_bias: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float* t = a.take<float>(n_out);
  SplitScratch sp;
  sp.floats = split_floats(TRINV_NB, n_out);
  sp.p = a.take<float>(sp.floats);
  RC(check_ws(a, "precondition_bias"));
  // t = Z_G^T g  (triangular.py:695/700), out = Z_G t  (triangular.py:696/701)
  RC(gemm(s, MATH_F32, n_out, 1, n_out, 1.0f, A_t(ZG, DT_F32, ldzg, TRI_LOWER), B_n(g, DT_F32, 1),
          0.0f, out_f32(t, 1), 1, sp));
  RC(gemm(s, MATH_F32, n_out, 1, n_out, 1.0f, A_n(ZG, DT_F32, ldzg, TRI_UPPER), B_n(t, DT_F32, 1),
          0.0f, out_f32(out, 1), 1, sp));
  return IFK_OK;
}

// ----------------------------------------------------------------------------
// bf16_linalg counterparts
// ----------------------------------------------------------------------------
size_t geqrf_r_ws(int64_t m, int64_t n) {
  Arena a(nullptr, 0);
  a.take<float>((size_t)n * n);
  FoldWs w;
  plan_fold(a, m, n, true, w);
  return a.used;
}

int geqrf_r(hipStream_t s, const void* A, int adt, int64_t m, int64_t n, int64_t lda, void* R,
            int rdt, int64_t ldr, int math, void* ws, size_t ws_bytes) {
  if (m < n || n < 1 || lda < n || ldr < n || !A || !R) {
    set_error("geqrf_r: invalid arguments (need m >= n >= 1)");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float* Rw = a.take<float>((size_t)n * n);
  FoldWs w;
  plan_fold(a, m, n, true, w);
  RC(check_ws(a, "geqrf_r"));
  RC(launch_zero(s, Rw, n, n, n));
  RC(launch_transpose_to_f32(s, A, adt, lda, m, n, w.C, m));
  RC(fold_core(s, w.C, m, m, n, Rw, n, n, false, math, w));
  return launch_cast_upper(s, Rw, n, n, R, rdt, ldr, nullptr);
}

size_t trsm_ws(int64_t n, int64_t k) {
  Arena a(nullptr, 0);
  a.take<float>((size_t)n * n);
  a.take<float>((size_t)n * n);
  float* tmp;
  SplitScratch sp;
  plan_trinv(a, std::max(n, k), &tmp, &sp);
  return a.used;
}

int trsm(hipStream_t s, const void* R, int rdt, int64_t n, int64_t ldr, int upper, const void* B,
         int bdt, int64_t k, int64_t ldb, void* X, int xdt, int64_t ldx, int math, void* ws,
         size_t ws_bytes) {
  if (n < 1 || k < 0 || ldr < n || (k > 0 && (ldb < k || ldx < k)) || !R || (k > 0 && (!B || !X))) {
    set_error("trsm: invalid arguments");
    return IFK_ERR_INVALID;
  }
  if (k == 0) return IFK_OK;
  Arena a(ws, ws_bytes);
  float* U = a.take<float>((size_t)n * n);
  float* Z = a.take<float>((size_t)n * n);
  float* tmp;
  SplitScratch sp;
  plan_trinv(a, std::max(n, k), &tmp, &sp);
  RC(check_ws(a, "trsm"));
  // Upper: X = R^{-1} B.  Lower: X = L^{-1} B = ((L^T)^{-1})^T B.
  if (upper) {
    RC(launch_copy_to_f32(s, R, rdt, ldr, n, n, 1.0f, U, n));
  } else {
    RC(launch_transpose_to_f32(s, R, rdt, ldr, n, n, U, n));
  }
  RC(trinv_core(s, U, DT_F32, n, n, Z, n, MATH_F32, 1, tmp, sp));
  const MatRef Aop = upper ? A_n(Z, DT_F32, n, TRI_UPPER) : A_t(Z, DT_F32, n, TRI_LOWER);
  const OutRef o = xdt == DT_BF16 ? out_bf16((bf16_t*)X, ldx) : out_f32((float*)X, ldx);
  return gemm(s, math, n, k, n, 1.0f, Aop, B_n(B, bdt, ldb), 0.0f, o, 1, sp);
}

static void plan_potrf(Arena& a, int64_t n, float** W, float** Zk, float** tmp, SplitScratch* sp) {
  *W = a.take<float>((size_t)n * n);
  *Zk = a.take<float>((size_t)TRINV_NB * TRINV_NB);
  *tmp = a.take<float>((size_t)TRINV_NB * n);
  sp->floats = split_floats(TRINV_NB, n);
  sp->p = a.take<float>(sp->floats);
}

size_t potrf_ws(int64_t n) {
  Arena a(nullptr, 0);
  float *W, *Zk, *tmp;
  SplitScratch sp;
  plan_potrf(a, n, &W, &Zk, &tmp, &sp);
  return a.used;
}

// Blocked right-looking upper Cholesky A = U^T U in the fp32 workspace W.
static int potrf_core(hipStream_t s, float* W, int64_t n, int math, float* Zk, float* tmp,
                      SplitScratch sp) {
  for (int64_t k0 = 0; k0 < n; k0 += TRINV_NB) {
    const int bk = (int)std::min<int64_t>(TRINV_NB, n - k0);
    const int64_t k1 = k0 + bk;
    float* Akk = W + k0 * n + k0;
    RC(launch_chol_block(s, Akk, n, bk));
    const int64_t nt = n - k1;
    if (nt > 0) {
      RC(launch_trinv_diag(s, Akk, DT_F32, n, bk, bk, Zk, bk, 1));
      // U[k, k1:] = U_kk^{-T} A[k, k1:]
      RC(gemm(s, MATH_F32, bk, nt, bk, 1.0f, A_t(Zk, DT_F32, bk, TRI_LOWER),
              B_n(W + k0 * n + k1, DT_F32, n), 0.0f, out_f32(tmp, nt), 1, sp));
      RC(launch_copy_to_f32(s, tmp, DT_F32, nt, bk, nt, 1.0f, W + k0 * n + k1, n));
      // A[k1:, k1:] -= U[k, k1:]^T U[k, k1:]
      RC(gemm(s, math, nt, nt, bk, -1.0f, A_t(tmp, DT_F32, nt), B_n(tmp, DT_F32, nt), 1.0f,
              out_f32(W + k1 * n + k1, n), 1, sp));
    }
  }
  return IFK_OK;
}

int potrf(hipStream_t s, const void* A, int adt, int64_t n, int64_t lda, void* L, int ldt,
          int64_t ldl, int math, void* ws, size_t ws_bytes) {
  if (n < 1 || lda < n || ldl < n || !A || !L) {
    set_error("potrf: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float *W, *Zk, *tmp;
  SplitScratch sp;
  plan_potrf(a, n, &W, &Zk, &tmp, &sp);
  RC(check_ws(a, "potrf"));
  RC(launch_copy_to_f32(s, A, adt, lda, n, n, 1.0f, W, n));
  RC(potrf_core(s, W, n, math, Zk, tmp, sp));
  return launch_transpose_upper(s, W, n, n, L, ldt, ldl);
}

size_t inv_spd_ws(int64_t n) {
  Arena a(nullptr, 0);
  float *W, *Zk, *tmp;
  SplitScratch sp;
  plan_potrf(a, n, &W, &Zk, &tmp, &sp);
  a.take<float>((size_t)n * n);
  float* ttmp;
  SplitScratch tsp;
  plan_trinv(a, n, &ttmp, &tsp);
  return a.used;
}

int inv_spd(hipStream_t s, const void* A, int adt, int64_t n, int64_t lda, void* X, int xdt,
            int64_t ldx, int math, void* ws, size_t ws_bytes) {
  if (n < 1 || lda < n || ldx < n || !A || !X) {
    set_error("inv_spd: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float *W, *Zk, *tmp;
  SplitScratch sp;
  plan_potrf(a, n, &W, &Zk, &tmp, &sp);
  float* Z = a.take<float>((size_t)n * n);
  float* ttmp;
  SplitScratch tsp;
  plan_trinv(a, n, &ttmp, &tsp);
  RC(check_ws(a, "inv_spd"));
  RC(launch_copy_to_f32(s, A, adt, lda, n, n, 1.0f, W, n));
  RC(potrf_core(s, W, n, math, Zk, tmp, sp));
  // A^{-1} = U^{-1} U^{-T} with A = U^T U  (bf16_linalg.py:275-279)
  RC(trinv_core(s, W, DT_F32, n, n, Z, n, MATH_F32, 1, ttmp, tsp));
  const OutRef o = xdt == DT_BF16 ? out_bf16((bf16_t*)X, ldx) : out_f32((float*)X, ldx);
  return gemm(s, math, n, n, n, 1.0f, A_n(Z, DT_F32, n, TRI_UPPER), B_t(Z, DT_F32, n, TRI_LOWER),
              0.0f, o, 1, tsp);
}

// ----------------------------------------------------------------------------
// Classic K-FAC control: explicit Gram factors and their damped inverses
// (ifkfac/kfac_hooks.py:208-258, ifkfac/classic_kfac.py:119-141, :218).
// ----------------------------------------------------------------------------
size_t gram_accumulate_ws(int64_t n) { return split_floats(TRINV_NB, n) * sizeof(float) + 256; }

int gram_accumulate(hipStream_t s, const void* X, int xdt, int64_t p, int64_t n, int64_t ldx,
                    float* S, int64_t lds, float beta, void* ws, size_t ws_bytes) {
  if (p < 1 || n < 1 || ldx < n || lds < n || !X || !S || (xdt != DT_F32 && xdt != DT_BF16)) {
    set_error("gram_accumulate: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  SplitScratch sp;
  sp.floats = split_floats(TRINV_NB, n);
  sp.p = a.take<float>(sp.floats);
  RC(check_ws(a, "gram_accumulate"));
  // the arithmetic of the activations' own product (torch mm in their dtype)
  const int math = xdt == DT_F32 ? MATH_F32 : MATH_BF16;
  RC(gemm(s, math, n, n, p, 1.0f, A_t(X, xdt, ldx), B_n(X, xdt, ldx), beta,
          lower_part(out_f32(S, lds)), 1, sp));
  return launch_mirror_lower(s, S, lds, n);
}

size_t inv_spd_damped_ws(int64_t n) { return inv_spd_ws(n); }

int inv_spd_damped(hipStream_t s, const void* A, int adt, int64_t n, int64_t lda, float damping,
                   float* X, int64_t ldx, void* ws, size_t ws_bytes) {
  if (n < 1 || lda < n || ldx < n || !A || !X || !(damping >= 0.0f)) {
    set_error("inv_spd_damped: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float *W, *Zk, *tmp;
  SplitScratch sp;
  plan_potrf(a, n, &W, &Zk, &tmp, &sp);
  float* Z = a.take<float>((size_t)n * n);
  float* ttmp;
  SplitScratch tsp;
  plan_trinv(a, n, &ttmp, &tsp);
  RC(check_ws(a, "inv_spd_damped"));
  RC(launch_copy_to_f32(s, A, adt, lda, n, n, 1.0f, W, n));
  RC(launch_add_diag(s, W, n, n, damping));
  RC(potrf_core(s, W, n, MATH_F32, Zk, tmp, sp));
  // (A + damping I)^{-1} = U^{-1} U^{-T} with A + damping I = U^T U
  RC(trinv_core(s, W, DT_F32, n, n, Z, n, MATH_F32, 1, ttmp, tsp));
  return gemm(s, MATH_F32, n, n, n, 1.0f, A_n(Z, DT_F32, n, TRI_UPPER),
              B_t(Z, DT_F32, n, TRI_LOWER), 0.0f, out_f32(X, ldx), 1, tsp);
}

size_t classic_precondition_ws(int64_t n_out, int64_t n_in) {
  return ((size_t)n_out * n_in + split_floats(TRINV_NB, std::max(n_out, n_in))) * sizeof(float) +
         512;
}

int classic_precondition(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in,
                         int64_t ldg, const float* A_inv, int64_t ldai, const float* G_inv,
                         int64_t ldgi, float* nat, int64_t ldn, void* ws, size_t ws_bytes) {
  if (n_out < 1 || n_in < 1 || ldg < n_in || ldai < n_in || ldgi < n_out || ldn < n_in || !grad ||
      !A_inv || !G_inv || !nat) {
    set_error("classic_precondition: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float* T = a.take<float>((size_t)n_out * n_in);
  SplitScratch sp;
  sp.floats = split_floats(TRINV_NB, std::max(n_out, n_in));
  sp.p = a.take<float>(sp.floats);
  RC(check_ws(a, "classic_precondition"));
  // nat = G^{-1} grad A^{-1} (classic_kfac.py:218), fp32 arithmetic
  RC(gemm(s, MATH_F32, n_out, n_in, n_in, 1.0f, A_n(grad, DT_F32, ldg), B_n(A_inv, DT_F32, ldai),
          0.0f, out_f32(T, n_in), 1, sp));
  return gemm(s, MATH_F32, n_out, n_in, n_out, 1.0f, A_n(G_inv, DT_F32, ldgi),
              B_n(T, DT_F32, n_in), 0.0f, out_f32(nat, ldn), 1, sp);
}

}  // namespace ifk
