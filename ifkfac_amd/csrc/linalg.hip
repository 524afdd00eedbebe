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
#include <cmath>

#include "gemm.h"
#include "kernels.h"
#include "linalg.h"

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
                      int64_t ldz, int math, int safe, float* tmp, SplitScratch sp);

struct FoldWs {
  float* C;      // p x n working copy of the chunk
  float* Yo;     // p x OUTER_B: reflector X parts of the current outer block
  float* Yto;    // p x OUTER_B: Y T of the outer block (fp32 arithmetic)
  bf16_t* Yob;   // bf16 copies of Yo, Y T and W for bf16 arithmetic (the
  bf16_t* Ytob;  // products round their operands to bf16 anyway)
  bf16_t* Wb;
  float* Q2;     // p x 64: X_p M1, or the fallback's reflectors
  float* W;      // OUTER_B x n
  float* part;   // per-slab Gram matrices of the panel kernels
  float* Gp;     // their sum: PANEL_MAX_CB blocks of 64 x 64
  float* NW;     // 64 x OUTER_B: N W of the panel
  float* U1;     // 64 x 64 panel scratch
  float* M1;
  float* Q1;
  float* N;
  float* NT;
  float* T;
  float* Go;     // OUTER_B x OUTER_B: Gram of the outer reflectors
  float* Tio;    // OUTER_B x OUTER_B: UT transform T^{-1}
  float* To;     // OUTER_B x OUTER_B: T of the outer block
  float* ttmp;   // triangular-inverse scratch for To
  SplitScratch tsp;
  int* flag;
  SplitScratch split;
};

static void plan_fold(Arena& a, int64_t p, int64_t n, bool need_C, FoldWs& w) {
  const int64_t b = PANEL_B, B = OUTER_B;
  w.C = need_C ? a.take<float>((size_t)p * n) : nullptr;
  w.Yo = a.take<float>((size_t)p * B);
  w.Yto = a.take<float>((size_t)p * B);
  w.Yob = a.take<bf16_t>((size_t)p * B);
  w.Ytob = a.take<bf16_t>((size_t)p * B);
  w.Wb = a.take<bf16_t>((size_t)B * n);
  w.Q2 = a.take<float>((size_t)p * b);
  w.W = a.take<float>((size_t)B * n);
  w.part = a.take<float>((size_t)gram_slabs(p) * PANEL_MAX_CB * b * b);
  w.Gp = a.take<float>((size_t)PANEL_MAX_CB * b * b);
  w.NW = a.take<float>((size_t)b * B);
  w.U1 = a.take<float>(b * b);
  w.M1 = a.take<float>(b * b);
  w.Q1 = a.take<float>(b * b);
  w.N = a.take<float>(b * b);
  w.NT = a.take<float>(b * b);
  w.T = a.take<float>(b * b);
  w.Go = a.take<float>(B * B);
  w.Tio = a.take<float>(B * B);
  w.To = a.take<float>(B * B);
  w.ttmp = a.take<float>((size_t)B * B / 2 + (size_t)TRINV_NB * TRINV_NB * 4);
  w.tsp.floats = split_floats(TRINV_NB, B);
  w.tsp.p = a.take<float>(w.tsp.floats);
  w.flag = a.take<int>(64);
  w.split.floats = split_floats(B, n);
  w.split.p = a.take<float>(w.split.floats);
}

// Apply the finished outer block (reflectors Yo of columns [K0, K1), pe rows)
// to the columns [K1, n):
//   T^{-1} = striu(Yo^T Yo) + diag(1 + diag(Yo^T Yo)) / 2   (UT transform)
//   W = (Yo T)^T C + T^T R_blk,  R_blk -= W,  C -= Yo W
// In bf16 arithmetic every product reads the bf16 copies (Yob, Ytob, Wb),
// which hold exactly the RNE roundings the MFMA operands would get; W and R
// stay fp32.
static int outer_update(hipStream_t s, int math, FoldWs& w, float* C, int64_t ldc, int64_t pe,
                        float* R, int64_t ldr, int64_t K0, int64_t K1, int64_t n) {
  const int64_t B = OUTER_B, KB = K1 - K0, nt = n - K1;
  const bool bf = math == MATH_BF16;
  const MatRef YoT = bf ? A_t(w.Yob, DT_BF16, B) : A_t(w.Yo, DT_F32, B);
  const MatRef YoB = bf ? B_n(w.Yob, DT_BF16, B) : B_n(w.Yo, DT_F32, B);
  RC(gemm(s, math, KB, KB, pe, 1.0f, YoT, YoB, 0.0f, out_f32(w.Go, KB), 1, w.split));
  RC(launch_ut_tinv(s, w.Go, KB, KB, w.Tio, KB));
  RC(trinv_core(s, w.Tio, DT_F32, KB, KB, w.To, KB, MATH_F32, 0, w.ttmp, w.tsp));
  const MatRef YoA = bf ? A_n(w.Yob, DT_BF16, B) : A_n(w.Yo, DT_F32, B);
  RC(gemm(s, math, pe, KB, KB, 1.0f, YoA, B_n(w.To, DT_F32, KB, TRI_UPPER), 0.0f,
          bf ? out_bf16(w.Ytob, B) : out_f32(w.Yto, B), 1, w.split));
  float* Rb = R + K0 * ldr + K1;
  const MatRef YtoT = bf ? A_t(w.Ytob, DT_BF16, B) : A_t(w.Yto, DT_F32, B);
  RC(gemm(s, math, KB, nt, pe, 1.0f, YtoT, B_n(C + K1, DT_F32, ldc), 0.0f, out_f32(w.W, nt), 1,
          w.split));
  RC(gemm(s, math, KB, nt, KB, 1.0f, A_t(w.To, DT_F32, KB, TRI_LOWER), B_n(Rb, DT_F32, ldr), 1.0f,
          bf ? out_both(w.W, nt, w.Wb, nt) : out_f32(w.W, nt), 1, w.split));
  RC(launch_sub_inplace(s, Rb, ldr, w.W, nt, KB, nt));
  const MatRef WB = bf ? B_n(w.Wb, DT_BF16, nt) : B_n(w.W, DT_F32, nt);
  return gemm(s, math, pe, nt, KB, -1.0f, YoA, WB, 1.0f, out_f32(C + K1, ldc), 1, w.split);
}

// Core of the fold on an fp32 working copy C (p x n, ldc).  R rows [0, r_new)
// receive the result.  Two-level blocking: 64-column panels inside 512-column
// outer blocks; a panel's reflectors update only the rest of its outer block,
// and each finished outer block is applied to the columns beyond it as one
// block reflector whose T is the UT transform of the outer Y.  With x_tri, C
// is upper triangular and a panel ending at column c1 involves C rows [0, c1).
static int fold_core(hipStream_t s, float* C, int64_t ldc, int64_t p, int64_t n, float* R,
                     int64_t ldr, int64_t r_new, bool x_tri, int math, FoldWs& w) {
  const int64_t B = OUTER_B;
  for (int64_t K0 = 0; K0 < r_new; K0 += B) {
    const int64_t K1 = std::min<int64_t>(K0 + B, r_new);
    const int64_t KB = K1 - K0;
    const int64_t pe_o = x_tri ? std::min<int64_t>(p, K1) : p;
    if (x_tri) {
      RC(launch_zero(s, w.Yo, B, pe_o, KB));
      if (math == MATH_BF16) RC(launch_zero_bf16(s, w.Yob, B, pe_o, KB));
    }
    for (int64_t c0 = K0; c0 < K1; c0 += PANEL_B) {
      const int bk = (int)std::min<int64_t>(PANEL_B, K1 - c0);
      const int64_t c1 = c0 + bk;
      const int nr = (int)(K1 - c1);
      const int64_t pe = x_tri ? std::min<int64_t>(p, c1) : p;
      float* Ptop = R + c0 * ldr + c0;
      float* Xp = C + c0;
      int ncb;
      // pass 1: G1 = X_p^T X_p (+ P_top^T P_top), U1, M1 -- or the fallback
      RC(launch_gram(s, Xp, ldc, bk, nullptr, 0, 0, Xp, ldc, bk, pe, w.part, w.Gp, &ncb));
      RC(launch_panel_hr_a(s, w.Gp, Ptop, ldr, bk, HR_TOL, w.U1, w.M1, w.Q1, w.flag));
      RC(launch_panel_hh_fallback(s, Ptop, ldr, Xp, ldc, pe, bk, w.Q2, w.flag));
      // pass 2: Q2 = X_p M1, G2 = Q2^T Q2 and Q2^T C_rest in one sweep
      RC(launch_apply_m(s, Xp, ldc, pe, bk, w.M1, w.Q2, w.flag));
      RC(launch_gram(s, w.Q2, PANEL_B, PANEL_B, w.Q2, PANEL_B, PANEL_B, C + c1, ldc, nr, pe, w.part,
                     w.Gp, &ncb));
      RC(launch_panel_hr_b(s, w.Gp, w.Q1, w.U1, bk, w.N, w.NT, w.T, Ptop, ldr, w.flag));
      // rest of the outer block: R_rest and C_rest, Y into the outer store
      RC(launch_panel_wcomp(s, w.Gp, ncb, bk, w.N, w.NT, w.T, Ptop + bk, ldr, nr, w.NW, OUTER_B));
      RC(launch_panel_update(s, w.Q2, pe, bk, w.N, w.Yo + (c0 - K0), OUTER_B,
                             math == MATH_BF16 ? w.Yob + (c0 - K0) : nullptr, w.NW, OUTER_B,
                             C + c1, ldc, nr));
    }
    if (K1 < n) RC(outer_update(s, math, w, C, ldc, pe_o, R, ldr, K0, K1, n));
  }
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
  RC(launch_copy_to_f32(s, X, xdt, ldx, p, n, 1.0f, w.C, n));
  RC(fold_core(s, w.C, n, p, n, R, ldr, r_new, false, math, w));
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
// Triangular inverse
// ----------------------------------------------------------------------------
static void plan_trinv(Arena& a, int64_t n, float** tmp, SplitScratch* sp) {
  *tmp = a.take<float>((size_t)n * n / 2 + (size_t)TRINV_NB * TRINV_NB * 4);
  sp->floats = split_floats(TRINV_NB, n);
  sp->p = a.take<float>(sp->floats);
}

size_t trinv_ws(int64_t n) {
  Arena a(nullptr, 0);
  float* tmp;
  SplitScratch sp;
  plan_trinv(a, n, &tmp, &sp);
  return a.used;
}

static int trinv_core(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z,
                      int64_t ldz, int math, int safe, float* tmp, SplitScratch sp) {
  const size_t esz = rdt == DT_F32 ? 4 : 2;
  const char* Rc = (const char*)R;
  RC(launch_zero(s, Z, ldz, n, n));
  RC(launch_trinv_diag(s, R, rdt, ldr, n, TRINV_NB, Z, ldz, safe));
  for (int64_t w = TRINV_NB; w < n; w *= 2) {
    const int64_t step = 2 * w;
    const int64_t nfull = n / step;
    if (nfull > 0) {
      const void* R12 = Rc + (size_t)w * esz;  // block (0, w)
      RC(gemm(s, math, w, w, w, 1.0f, A_n(R12, rdt, ldr, TRI_NONE, step * (ldr + 1)),
              B_n(Z + w * ldz + w, DT_F32, ldz, TRI_UPPER, step * (ldz + 1)), 0.0f,
              out_f32(tmp, w, w * w), (int)nfull, sp));
      RC(gemm(s, math, w, w, w, -1.0f, A_n(Z, DT_F32, ldz, TRI_UPPER, step * (ldz + 1)),
              B_n(tmp, DT_F32, w, TRI_NONE, w * w), 0.0f, out_f32(Z + w, ldz, step * (ldz + 1)),
              (int)nfull, sp));
    }
    const int64_t i0 = nfull * step;
    if (i0 + w < n) {
      const int64_t w2 = n - i0 - w;
      const void* R12 = Rc + ((size_t)i0 * ldr + i0 + w) * esz;
      RC(gemm(s, math, w, w2, w, 1.0f, A_n(R12, rdt, ldr),
              B_n(Z + (i0 + w) * ldz + i0 + w, DT_F32, ldz, TRI_UPPER), 0.0f, out_f32(tmp, w2), 1,
              sp));
      RC(gemm(s, math, w, w2, w, -1.0f, A_n(Z + i0 * ldz + i0, DT_F32, ldz, TRI_UPPER),
              B_n(tmp, DT_F32, w2), 0.0f, out_f32(Z + i0 * ldz + i0 + w, ldz), 1, sp));
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
  SplitScratch sp;
  plan_trinv(a, n, &tmp, &sp);
  RC(check_ws(a, "tri_inverse"));
  return trinv_core(s, R, rdt, ldr, n, Z, ldz, math, safe, tmp, sp);
}

// ----------------------------------------------------------------------------
// Preconditioning
// ----------------------------------------------------------------------------
static void plan_apply(Arena& a, int64_t n_out, int64_t n_in, int math, void** T1, void** T2,
                       SplitScratch* sp) {
  const size_t e = (size_t)n_out * n_in;
  if (math == MATH_BF16) {
    *T1 = a.take<bf16_t>(e);
    *T2 = a.take<bf16_t>(e);
  } else {
    *T1 = a.take<float>(e);
    *T2 = a.take<float>(e);
  }
  sp->floats = split_floats(TRINV_NB, std::max(n_out, n_in));
  sp->p = a.take<float>(sp->floats);
}

size_t precondition_apply_ws(int64_t n_out, int64_t n_in, int math) {
  Arena a(nullptr, 0);
  void *T1, *T2;
  SplitScratch sp;
  plan_apply(a, n_out, n_in, math, &T1, &T2, &sp);
  return a.used;
}

static int apply_core(hipStream_t s, const float* grad, int64_t n_out, int64_t n_in, int64_t ldg,
                      const float* ZX, int64_t ldzx, const float* ZG, int64_t ldzg, float* nat,
                      int64_t ldn, int math, void* T1, void* T2, SplitScratch sp) {
  const int tdt = math == MATH_BF16 ? DT_BF16 : DT_F32;
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
  SplitScratch sp;
  plan_apply(a, n_out, n_in, math, &T1, &T2, &sp);
  RC(check_ws(a, "precondition_apply"));
  return apply_core(s, grad, n_out, n_in, ldg, ZX, ldzx, ZG, ldzg, nat, ldn, math, T1, T2, sp);
}

static void plan_prec(Arena& a, int64_t n_out, int64_t n_in, int math, float** ZX, float** ZG,
                      float** tmp, SplitScratch* tsp, void** T1, void** T2, SplitScratch* asp) {
  *ZX = a.take<float>((size_t)n_in * n_in);
  *ZG = a.take<float>((size_t)n_out * n_out);
  plan_trinv(a, std::max(n_in, n_out), tmp, tsp);
  plan_apply(a, n_out, n_in, math, T1, T2, asp);
}

size_t precondition_ws(int64_t n_out, int64_t n_in, int math) {
  Arena a(nullptr, 0);
  float *ZX, *ZG, *tmp;
  void *T1, *T2;
  SplitScratch tsp, asp;
  plan_prec(a, n_out, n_in, math, &ZX, &ZG, &tmp, &tsp, &T1, &T2, &asp);
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
  void *T1, *T2;
  SplitScratch tsp, asp;
  plan_prec(a, n_out, n_in, math, &ZX, &ZG, &tmp, &tsp, &T1, &T2, &asp);
  RC(check_ws(a, "precondition"));
  RC(trinv_core(s, RX, rdt, ldrx, n_in, ZX, n_in, math, 0, tmp, tsp));
  RC(trinv_core(s, RG, rdt, ldrg, n_out, ZG, n_out, math, 0, tmp, tsp));
  return apply_core(s, grad, n_out, n_in, ldg, ZX, n_in, ZG, n_out, nat, ldn, math, T1, T2, asp);
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
  RC(launch_copy_to_f32(s, A, adt, lda, m, n, 1.0f, w.C, n));
  RC(fold_core(s, w.C, n, m, n, Rw, n, n, false, math, w));
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

}  // namespace ifk
