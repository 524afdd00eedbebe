// Single-workgroup kernels on b x b (b <= 64) matrices held in LDS, used by the
// panel factorisation of the streaming fold and by the blocked triangular
// inverse and Cholesky.  Matrices are fp32, padded to 64 x 64 with the
// identity beyond b, row stride SLD.  Dense 64-wide work is blocked in 16 x 16
// tiles: a diagonal tile is factored or inverted in registers by 16 lanes of
// one wave (values exchanged with v_readlane broadcasts), off-diagonal tiles
// by LDS products, so a 64 x 64 Cholesky or inverse needs about a dozen
// workgroup barriers instead of one or more per column.
//
// Panel of the fold (columns [c0, c0+b) of the stacked [R; X]):
//   P = [P_top; X_p], P_top the b x b upper-triangular diagonal block of R,
//   X_p the p_e x b block of the working X.
// Reflectors come from CholeskyQR2 plus Householder reconstruction:
//   G1 = P^T P = U1^T U1, M1 = U1^{-1}, Q = P M1                 (panel_hr_a)
//   G2 = Q^T Q = U2^T U2, M2 = U2^{-1}, Q_f = Q M2               (panel_hrw)
//   S = diag(-sign((Q_f,top)_jj)), T = I - Q_f,top S (upper triangular)
//   Y = Q_bottom N with N = -M2 S T^{-1},  Y T = Q_bottom (-M2 S)
//   R_new = S U2 U1
// which is the TPQRT form: V = [I; Y], block reflector I - V T V^T.  When a
// first-pass Cholesky pivot collapses (rank-deficient or ill-conditioned
// panel) a flag is raised and the Householder fallback (panel_fallback.h, run by
// apply_m in place of Q2 = X_p M1) computes the reflectors by
// column-by-column Householder reflections (LAPACK dlarfg convention, never
// breaks down); panel_hrw then takes T from the UT transform
//   T^{-1} = striu(V^T V) + diag(V^T V) / 2,  V^T V = I + Y^T Y.
// The partial Gram matrices over row slabs come from panel.hip.
#include "common.h"
#include "kernels.h"

namespace ifk {

constexpr int SB = 64;        // max panel / block width
constexpr int SLD = SB + 1;   // LDS row stride (floats)
constexpr int SNT = 256;
constexpr int TB = 16;        // register tile

__device__ inline float bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// ---------------------------------------------------------------------------
// LDS building blocks (all called by the whole 256-thread workgroup)
// ---------------------------------------------------------------------------

// Load a b x b block (row stride ld) into a padded 64 x 64 LDS matrix.  With
// upper set, the strict lower part is zeroed.  The pad beyond b is pad * I.
__device__ __forceinline__ void sm_load_pad(float* S, const float* g, int64_t ld, int b, bool upper,
                                            float pad = 1.0f) {
  // every load of the thread is issued before the first LDS write, so the
  // 16 loads share one memory latency
  constexpr int PER = SB * SB / SNT;
  float v[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = threadIdx.x + SNT * q;
    const int r = e >> 6, c = e & 63;
    if (r < b && c < b) v[q] = (upper && r > c) ? 0.0f : g[(int64_t)r * ld + c];
    else v[q] = (r == c) ? pad : 0.0f;
  }
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = threadIdx.x + SNT * q;
    S[(e >> 6) * SLD + (e & 63)] = v[q];
  }
  __syncthreads();
}

// C = alpha * op(A) op(B) (+ C if acc) for padded 64 x 64 LDS matrices, with
// op(X) = X^T when the flag is set, on fp32 MFMA: wave w computes the 32 x 32
// quadrant (w >> 1, w & 1) of C with 32 v_mfma_f32_32x32x2f32 (lane (l32, h)
// supplies k = 32 h + s to step s).  Zeros of triangular operands are
// multiplied like any other value.  C may alias A or B: every read completes
// before the first write.
template <bool TA, bool TBt>
__device__ __forceinline__ void sm_gemm64(const float* A, const float* B, float* C, float alpha,
                                          bool acc) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int r = (wave >> 1) * 32 + l32;   // row of op(A) this lane supplies
  const int c = (wave & 1) * 32 + l32;    // column of op(B) this lane supplies
  f32x16 d;
#pragma unroll
  for (int i = 0; i < 16; ++i) d[i] = 0.0f;
#pragma unroll
  for (int s = 0; s < 32; ++s) {
    const int k = 32 * h + s;
    const float a = TA ? A[k * SLD + r] : A[r * SLD + k];
    const float b = TBt ? B[c * SLD + k] : B[k * SLD + c];
    d = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, d, 0, 0, 0);
  }
  __syncthreads();
  const int row0 = (wave >> 1) * 32, col = (wave & 1) * 32 + l32;
  float cur[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    cur[i] = acc ? C[(row0 + (i >> 2) * 8 + h * 4 + (i & 3)) * SLD + col] : 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    C[(row0 + (i >> 2) * 8 + h * 4 + (i & 3)) * SLD + col] = cur[i] + alpha * d[i];
  __syncthreads();
}

__device__ __forceinline__ void sm_store(const float* S, float* g, int64_t ld, int b) {
  for (int e = threadIdx.x; e < b * b; e += SNT) {
    const int r = e / b, c = e - r * b;
    g[(int64_t)r * ld + c] = S[r * SLD + c];
  }
}

// Divisor rule of bf16_linalg._safe_div (bf16_linalg.py:44-59): a magnitude
// below 1e-7 is replaced by sign(d) * 1e-7 with sign(0) = +1.
__device__ inline float safe_divisor(float d) {
  return fabsf(d) < 1e-7f ? (d < 0.0f ? -1e-7f : 1e-7f) : d;
}

// Upper Cholesky in place (A = U^T U, upper triangle read, strict lower
// zeroed on exit).  mode 0: a pivot below tol * (its diagonal on entry) or not
// finite raises *bad (the factorisation continues on a clamped pivot so every
// thread runs the same steps); mode 1: the pivot rule of cholesky_bf16,
// max(pivot, 1e-7).
//
// Right-looking, blocked by CB = 8 columns.  Every thread factors the 8 x 8
// diagonal block and inverts it redundantly in registers (no cross-lane
// traffic on the sequential chain), then owns one column of the block row
// (U_kr = W_kk^T A_kr with W_kk = U_kk^{-1}) and finally a column of the
// rank-8 trailing update.  Three barriers per block.
__device__ __forceinline__ void sm_chol64(float* A, float tol, int* bad, int mode) {
  constexpr int CB = 8;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  __shared__ float dg[SB];
  for (int j = t; j < SB; j += SNT) dg[j] = A[j * SLD + j];
  __syncthreads();
  int flag = 0;
  for (int kb = 0; kb < SB / CB; ++kb) {
    const int o = kb * CB;
    float u[CB][CB], w[CB][CB];
#pragma unroll
    for (int i = 0; i < CB; ++i)
#pragma unroll
      for (int j = i; j < CB; ++j) u[i][j] = A[(o + i) * SLD + o + j];
    __syncthreads();  // every read of the diagonal block precedes its overwrite
#pragma unroll
    for (int k = 0; k < CB; ++k) {
      const float piv = u[k][k];
      float pv, rs;
      if (mode == 0) {
        if (!(piv > tol * dg[o + k]) || !isfinite(piv)) flag = 1;
        pv = fmaxf(piv, 1e-30f);
        rs = __builtin_amdgcn_rsqf(pv);
        u[k][k] = pv * rs;
      } else {
        pv = fmaxf(piv, 1e-7f);
        u[k][k] = sqrtf(pv);
        rs = 1.0f / u[k][k];
      }
      w[k][k] = rs;
#pragma unroll
      for (int j = k + 1; j < CB; ++j) u[k][j] *= rs;
#pragma unroll
      for (int i = k + 1; i < CB; ++i)
#pragma unroll
        for (int j = i; j < CB; ++j) u[i][j] = fmaf(-u[k][i], u[k][j], u[i][j]);
    }
    // W = U_kk^{-1}, column by column (upper triangular)
#pragma unroll
    for (int j = 1; j < CB; ++j)
#pragma unroll
      for (int i = j - 1; i >= 0; --i) {
        float s = 0.0f;
#pragma unroll
        for (int k = i + 1; k <= j; ++k) s = fmaf(u[i][k], w[k][j], s);
        w[i][j] = -s * w[i][i];
      }
    if (t < CB * CB) {
      const int i = t / CB, j = t % CB;
      float v = 0.0f;
#pragma unroll
      for (int a = 0; a < CB; ++a)
#pragma unroll
        for (int b = a; b < CB; ++b)
          if (a == i && b == j) v = u[a][b];
      A[(o + i) * SLD + o + j] = v;
    }
    // block row: U[o:o+CB, c] = W^T A[o:o+CB, c]
    const int c = o + CB + t;
    if (c < SB) {
      float x[CB];
#pragma unroll
      for (int i = 0; i < CB; ++i) x[i] = A[(o + i) * SLD + c];
#pragma unroll
      for (int i = 0; i < CB; ++i) {
        float s = 0.0f;
#pragma unroll
        for (int m = 0; m <= i; ++m) s = fmaf(w[m][i], x[m], s);
        A[(o + i) * SLD + c] = s;
      }
    }
    __syncthreads();
    // rank-CB trailing update A[r][c] -= sum_k U[o+k][r] U[o+k][c] for
    // r, c >= o + CB on fp32 MFMA: wave w takes the 32 x 32 quadrant
    // (w >> 1, w & 1); lane (l32, h) supplies k = 4 h + s to step s.  The
    // strictly lower quadrant and quadrants left of the block are skipped;
    // within a quadrant the lower-triangle results are discarded.
    {
      typedef float f32x16 __attribute__((ext_vector_type(16)));
      const int lo = o + CB;
      const int q0 = (wave >> 1) * 32, q1 = (wave & 1) * 32;
      if (wave != 2 && q0 + 31 >= lo && q1 + 31 >= lo) {
        const int l32 = lane & 31, h = lane >> 5;
        const int r = q0 + l32, c = q1 + l32;
        f32x16 d;
#pragma unroll
        for (int i = 0; i < 16; ++i) d[i] = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < CB / 2; ++s2) {
          const int k = o + (CB / 2) * h + s2;
          const float a = (r >= lo) ? A[k * SLD + r] : 0.0f;
          const float b = (c >= lo) ? A[k * SLD + c] : 0.0f;
          d = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, d, 0, 0, 0);
        }
        // all reads before any write, so the 16 updates share one LDS latency
        float cur[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) cur[i] = A[(q0 + (i >> 2) * 8 + h * 4 + (i & 3)) * SLD + c];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int row = q0 + (i >> 2) * 8 + h * 4 + (i & 3);
          if (row >= lo && c >= row) A[row * SLD + c] = cur[i] - d[i];
        }
      }
    }
    __syncthreads();
  }
  for (int e = t; e < SB * SB; e += SNT) {
    const int r = e >> 6, cc = e & 63;
    if (r > cc) A[r * SLD + cc] = 0.0f;
  }
  if (t == 0 && flag && bad) *bad = 1;
  __syncthreads();
}

// Z = U^{-1} for a padded 64 x 64 upper-triangular U (Z strict lower = 0).
// Tmp: LDS scratch of 32 * 32 floats.  With safe set, diagonal divisors follow
// safe_divisor.
__device__ __forceinline__ void sm_trinv64(const float* U, float* Z, float* Tmp, bool safe = false) {
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  for (int e = t; e < SB * SB; e += SNT) Z[(e >> 6) * SLD + (e & 63)] = 0.0f;
  __syncthreads();
  // 1) the four diagonal 16 x 16 tiles, one wave each, one lane per column
  {
    const int o = wave * TB;
    if (lane < TB) {
      float z[TB], rd[TB];
#pragma unroll
      for (int i = 0; i < TB; ++i) {
        const float d = U[(o + i) * SLD + o + i];
        rd[i] = 1.0f / (safe ? safe_divisor(d) : d);  // independent of the chain below
      }
#pragma unroll
      for (int i = TB - 1; i >= 0; --i) {
        float s = (i == lane) ? 1.0f : 0.0f;
#pragma unroll
        for (int k = i + 1; k < TB; ++k) s = fmaf(-U[(o + i) * SLD + o + k], z[k], s);
        z[i] = s * rd[i];
      }
#pragma unroll
      for (int i = 0; i < TB; ++i) Z[(o + i) * SLD + o + lane] = z[i];
    }
  }
  __syncthreads();
  // 2) level 16: Z_01 = -Z_00 U_01 Z_11 for tile pairs (0,1) and (2,3)
  for (int e = t; e < 2 * TB * TB; e += SNT) {
    const int pr = e / (TB * TB), w = e % (TB * TB);
    const int i = w / TB, j = w % TB;
    const int o0 = pr * 2 * TB, o1 = o0 + TB;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < TB; ++k) s += U[(o0 + i) * SLD + o1 + k] * Z[(o1 + k) * SLD + o1 + j];
    Tmp[pr * TB * TB + i * TB + j] = s;
  }
  __syncthreads();
  for (int e = t; e < 2 * TB * TB; e += SNT) {
    const int pr = e / (TB * TB), w = e % (TB * TB);
    const int i = w / TB, j = w % TB;
    const int o0 = pr * 2 * TB, o1 = o0 + TB;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < TB; ++k) s += Z[(o0 + i) * SLD + o0 + k] * Tmp[pr * TB * TB + k * TB + j];
    Z[(o0 + i) * SLD + o1 + j] = -s;
  }
  __syncthreads();
  // 3) level 32: Z[0:32, 32:64] = -Z[0:32, 0:32] U[0:32, 32:64] Z[32:64, 32:64]
  // (the zero lower triangles are part of the unrolled products)
  for (int e = t; e < 32 * 32; e += SNT) {
    const int i = e >> 5, j = e & 31;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; ++k) s = fmaf(U[i * SLD + 32 + k], Z[(32 + k) * SLD + 32 + j], s);
    Tmp[i * 32 + j] = s;
  }
  __syncthreads();
  for (int e = t; e < 32 * 32; e += SNT) {
    const int i = e >> 5, j = e & 31;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; ++k) s = fmaf(Z[i * SLD + k], Tmp[k * 32 + j], s);
    Z[i * SLD + 32 + j] = -s;
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Panel kernels
// ---------------------------------------------------------------------------

// CholeskyQR pass 1.  In: G = X_p^T X_p (64 x 64, ld 64), P_top (in R at ldr).
// Out: U1 (Cholesky factor of P^T P), M1 = U1^{-1}, Q1 = P_top M1 (b x b,
// ld b); *flag = 1 when a pivot falls below tol times its diagonal (the
// panel then goes to the Householder fallback), else 0.
__global__ __launch_bounds__(SNT) void panel_hr_a_kernel(const float* G,
                                                          const float* Ptop, int64_t ldr, int b,
                                                          float tol, float* U1, float* M1,
                                                          float* Q1, int* flag) {
  __shared__ float sG[SB * SLD];
  __shared__ float sP[SB * SLD];
  __shared__ float sM[SB * SLD];
  __shared__ float sT[32 * 32];
  __shared__ int bad;
  if (threadIdx.x == 0) bad = 0;
  sm_load_pad(sG, G, SB, b, false);
  sm_load_pad(sP, Ptop, ldr, b, true, 0.0f);
  sm_gemm64<true, false>(sP, sP, sG, 1.0f, true);  // sG = X_p^T X_p + P_top^T P_top
  sm_chol64(sG, tol, &bad, 0);                     // sG = U1
  sm_store(sG, U1, b, b);
  sm_trinv64(sG, sM, sT);                          // sM = M1
  sm_store(sM, M1, b, b);
  sm_gemm64<false, false>(sP, sM, sG, 1.0f, false);  // sG = Q1 = P_top M1
  sm_store(sG, Q1, b, b);
  __syncthreads();
  if (threadIdx.x == 0) *flag = bad;
}

// CholeskyQR pass 2, Householder reconstruction and the update of the rest of
// the outer block, one launch of 1 + nblk workgroups.  In: G[0] = G2 =
// Q2^T Q2 and G[1 + cb] = Q2^T C_rest block cb (64 x 64 each, ld 64;
// Q2 = X_p M1), Q1, U1.  Every workgroup builds T, NT (Y T = Q2 NT) and N
// (Y = Q2 N) in LDS -- the redundant 64 x 64 work costs no time on the
// critical path, and it saves a launch and a round trip through memory.
//   workgroup 0:      N to global; R's diagonal block <- R_new = S U2 U1
//   workgroup 1 + cb: W = NT^T (Q2^T C) + T^T R_rest, R_rest -= W, NW = N W
//                     for the 64-column block cb of R_rest (nr columns)
// For a panel flagged by pass 1, Q2 holds the fallback's reflectors Y and R
// already holds R_new: T comes from the UT transform of Y^T Y, N = I, NT = T.
// A second-pass pivot below 1/4 (the first pass lost too much orthogonality
// for the reconstruction to be exact) poisons R's block with NaN, which the
// finite check of finalize reports.
__global__ __launch_bounds__(SNT) void panel_hrw_kernel(const float* G, const float* Q1,
                                                         const float* U1, int b, float* N,
                                                         float* R, int64_t ldr, int nr,
                                                         float* NW, int64_t ldnw,
                                                         const int* flag) {
  __shared__ float sG[SB * SLD];
  __shared__ float sQ[SB * SLD];
  __shared__ float sM[SB * SLD];
  __shared__ float sX[SB * SLD];
  __shared__ float sN[SB * SLD];
  __shared__ float sTmp[32 * 32];
  __shared__ float sgn[SB];
  __shared__ int bad;
  const int t = threadIdx.x;
  const int role = blockIdx.x;   // 0: R_new and N; 1 + cb: block cb of the rest
  if (t == 0) bad = 0;
  const bool flagged = (*flag != 0);
  sm_load_pad(sG, G, SB, b, false);
  if (flagged) {
    // UT transform: T^{-1} = striu(Y^T Y) + diag(1 + diag(Y^T Y)) / 2
    for (int e = t; e < SB * SB; e += SNT) {
      const int i = e >> 6, j = e & 63;
      float v = 0.0f;
      if (i < b && j < b) {
        if (i < j) v = sG[i * SLD + j];
        else if (i == j) v = 0.5f * (1.0f + sG[i * SLD + i]);
      } else if (i == j) {
        v = 1.0f;
      }
      sM[i * SLD + j] = v;
    }
    __syncthreads();
    sm_trinv64(sM, sX, sTmp);                        // sX = T
    for (int e = t; e < SB * SB; e += SNT) {
      const int i = e >> 6, j = e & 63;
      const float id = (i == j) ? 1.0f : 0.0f;
      sN[i * SLD + j] = id;                          // N = I
      sQ[i * SLD + j] = sX[i * SLD + j];             // NT = T
    }
    __syncthreads();
  } else {
    sm_load_pad(sQ, Q1, b, b, true, 0.0f);
    sm_gemm64<true, false>(sQ, sQ, sG, 1.0f, true);  // sG = Q2^T Q2 + Q1^T Q1
    sm_chol64(sG, 0.25f, &bad, 0);                   // sG = U2
    sm_trinv64(sG, sM, sTmp);                        // sM = M2
    sm_gemm64<false, false>(sQ, sM, sX, 1.0f, false);  // sX = Q1f = Q1 M2
    for (int j = t; j < SB; j += SNT) sgn[j] = (sX[j * SLD + j] >= 0.0f) ? -1.0f : 1.0f;
    __syncthreads();
    // sX <- T = I - Q1f S (upper triangular; identity in the pad)
    for (int e = t; e < SB * SB; e += SNT) {
      const int i = e >> 6, j = e & 63;
      float v = (i == j) ? 1.0f : 0.0f;
      if (i < b && j < b && i <= j) v -= sX[i * SLD + j] * sgn[j];
      sX[i * SLD + j] = v;
    }
    __syncthreads();
    sm_trinv64(sX, sQ, sTmp);                        // sQ = T^{-1}
    for (int e = t; e < SB * SB; e += SNT) {         // sQ <- S T^{-1}
      const int k = e >> 6, j = e & 63;
      sQ[k * SLD + j] *= sgn[k];
    }
    __syncthreads();
    sm_gemm64<false, false>(sM, sQ, sN, -1.0f, false);  // sN = N = -M2 S T^{-1}
    for (int e = t; e < SB * SB; e += SNT) {         // sQ <- NT = -M2 S (zero in the pad)
      const int i = e >> 6, j = e & 63;
      sQ[i * SLD + j] = (i < b && j < b) ? -sM[i * SLD + j] * sgn[j] : 0.0f;
    }
    __syncthreads();
  }
  // here: sX = T, sQ = NT, sN = N (all zero / identity beyond b as built)
  if (role == 0) {
    for (int e = t; e < b * b; e += SNT) {
      const int i = e / b, j = e - i * b;
      N[e] = sN[i * SLD + j];
    }
    if (flagged) return;
    const bool ok = (bad == 0);
    sm_load_pad(sM, U1, b, b, true);
    sm_gemm64<false, false>(sG, sM, sM, 1.0f, false);  // sM = U2 U1
    const float nan = __int_as_float(0x7fc00000);
    for (int e = t; e < b * b; e += SNT) {           // R_new = S U2 U1
      const int i = e / b, j = e - i * b;
      R[(int64_t)i * ldr + j] = !ok ? nan : ((i <= j) ? sgn[i] * sM[i * SLD + j] : 0.0f);
    }
    return;
  }
  // block cb of the rest: columns [b + c0, b + c0 + w) of R's block row
  const int cb = role - 1;
  const int c0 = cb * SB;
  const int w = (nr - c0) < SB ? (nr - c0) : SB;
  float* Rrest = R + b;
  sm_load_pad(sG, G + (size_t)(1 + cb) * SB * SB, SB, SB, false);  // Q2^T C block
  sm_gemm64<true, false>(sQ, sG, sM, 1.0f, false);     // sM = W = NT^T (Q2^T C)
  {
    float v[SB * SB / SNT];
#pragma unroll
    for (int q = 0; q < SB * SB / SNT; ++q) {
      const int e = t + SNT * q, i = e >> 6, j = e & 63;
      v[q] = (i < b && j < w) ? Rrest[(int64_t)i * ldr + c0 + j] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < SB * SB / SNT; ++q) {
      const int e = t + SNT * q;
      sG[(e >> 6) * SLD + (e & 63)] = v[q];
    }
  }
  __syncthreads();
  sm_gemm64<true, false>(sX, sG, sM, 1.0f, true);      // W += T^T R_rest
  for (int e = t; e < SB * SB; e += SNT) {
    const int i = e >> 6, j = e & 63;
    if (i < b && j < w) Rrest[(int64_t)i * ldr + c0 + j] = sG[i * SLD + j] - sM[i * SLD + j];
  }
  sm_gemm64<false, false>(sN, sM, sG, 1.0f, false);    // NW = N W
  for (int e = t; e < SB * SB; e += SNT) {
    const int i = e >> 6, j = e & 63;
    NW[(int64_t)i * ldnw + c0 + j] = sG[i * SLD + j];
  }
}

// ---------------------------------------------------------------------------
// Diagonal block of a blocked upper Cholesky (bf16_linalg.cholesky_bf16 pivot
// rule, bf16_linalg.py:258-260): U_jj = sqrt(max(A_jj - sum_k U_kj^2, 1e-7)).
// In place on a b x b block at A (ld); only the upper triangle is read; on
// exit the block holds U (strict lower part zeroed).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(SNT) void chol_block_kernel(float* A, int64_t ld, int b) {
  __shared__ float sA[SB * SLD];
  sm_load_pad(sA, A, ld, b, true);
  sm_chol64(sA, 0.0f, nullptr, 1);
  for (int e = threadIdx.x; e < b * b; e += SNT) {
    const int r = e / b, c = e - r * b;
    A[(int64_t)r * ld + c] = (r <= c) ? sA[r * SLD + c] : 0.0f;
  }
}

// UT transform: T^{-1} = striu(G) + diag(1 + diag G) / 2 for a Gram matrix G.
__global__ void ut_tinv_kernel(const float* G, int64_t ldg, int64_t n, float* Tinv, int64_t ldt) {
  const int64_t total = n * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / n, j = e % n;
    float v = 0.0f;
    if (i < j) v = G[i * ldg + j];
    else if (i == j) v = 0.5f * (1.0f + G[i * ldg + i]);
    Tinv[i * ldt + j] = v;
  }
}

// ---------------------------------------------------------------------------
// Diagonal blocks of a blocked triangular inverse: Z_kk = R_kk^{-1} for every
// nb x nb block on the diagonal of an upper-triangular R (last block may be
// ragged).  One workgroup per block.
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(SNT) void trinv_diag_kernel(const void* R, int64_t ldr, int64_t n,
                                                         int nb, float* Z, int64_t ldz, int safe) {
  __shared__ float sU[SB * SLD];
  __shared__ float sZ[SB * SLD];
  __shared__ float sT[32 * 32];
  const int64_t k0 = (int64_t)blockIdx.x * nb;
  const int b = (int)((n - k0) < nb ? (n - k0) : nb);
  {
    float v[SB * SB / SNT];
#pragma unroll
    for (int q = 0; q < SB * SB / SNT; ++q) {
      const int e = threadIdx.x + SNT * q, r = e >> 6, c = e & 63;
      if (r < b && c < b)
        v[q] = (r <= c)
                   ? Elem<DT>::load((const typename Elem<DT>::T*)R + (k0 + r) * ldr + k0 + c)
                   : 0.0f;
      else
        v[q] = (r == c) ? 1.0f : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < SB * SB / SNT; ++q) {
      const int e = threadIdx.x + SNT * q;
      sU[(e >> 6) * SLD + (e & 63)] = v[q];
    }
  }
  __syncthreads();
  sm_trinv64(sU, sZ, sT, safe != 0);
  for (int e = threadIdx.x; e < b * b; e += SNT) {
    const int r = e / b, c = e - r * b;
    Z[(k0 + r) * ldz + k0 + c] = sZ[r * SLD + c];
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
static int check_b(int b, const char* what) {
  if (b > SB || b < 1) {
    set_error(std::string(what) + ": block size out of range");
    return IFK_ERR_INVALID;
  }
  return IFK_OK;
}

int launch_panel_hr_a(hipStream_t s, const float* G, const float* Ptop, int64_t ldr, int b,
                      float tol, float* U1, float* M1, float* Q1, int* flag) {
  if (int rc = check_b(b, "panel_hr_a")) return rc;
  hipLaunchKernelGGL(panel_hr_a_kernel, dim3(1), dim3(SNT), 0, s, G, Ptop, ldr, b, tol, U1, M1, Q1,
                     flag);
  return check_launch("panel_hr_a");
}

int launch_panel_hrw(hipStream_t s, const float* G, int ncb, const float* Q1, const float* U1,
                     int b, float* N, float* R, int64_t ldr, int nr, float* NW, int64_t ldnw,
                     const int* flag) {
  if (int rc = check_b(b, "panel_hrw")) return rc;
  const int nblk = nr > 0 ? (int)cdiv((int64_t)nr, (int64_t)SB) : 0;
  if (ncb != nblk + 1 || (nblk > 0 && ldnw < (int64_t)nblk * SB)) {
    set_error("panel_hrw: column blocks do not match the partial Grams");
    return IFK_ERR_INVALID;
  }
  hipLaunchKernelGGL(panel_hrw_kernel, dim3(1 + nblk), dim3(SNT), 0, s, G, Q1, U1, b, N, R, ldr, nr,
                     NW, ldnw, flag);
  return check_launch("panel_hrw");
}

int launch_chol_block(hipStream_t s, float* A, int64_t ld, int b) {
  if (int rc = check_b(b, "chol_block")) return rc;
  hipLaunchKernelGGL(chol_block_kernel, dim3(1), dim3(SNT), 0, s, A, ld, b);
  return check_launch("chol_block");
}

int launch_ut_tinv(hipStream_t s, const float* G, int64_t ldg, int64_t n, float* Tinv,
                   int64_t ldt) {
  if (n == 0) return IFK_OK;
  int64_t g = cdiv(n * n, 256);
  if (g > 4096) g = 4096;
  hipLaunchKernelGGL(ut_tinv_kernel, dim3((unsigned)g), dim3(256), 0, s, G, ldg, n, Tinv, ldt);
  return check_launch("ut_tinv");
}

int launch_trinv_diag(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, int nb,
                      float* Z, int64_t ldz, int safe) {
  if (int rc = check_b(nb, "trinv_diag")) return rc;
  const unsigned nblk = (unsigned)cdiv(n, nb);
  if (rdt == DT_F32)
    hipLaunchKernelGGL(trinv_diag_kernel<DT_F32>, dim3(nblk), dim3(SNT), 0, s, R, ldr, n, nb, Z,
                       ldz, safe);
  else
    hipLaunchKernelGGL(trinv_diag_kernel<DT_BF16>, dim3(nblk), dim3(SNT), 0, s, R, ldr, n, nb, Z,
                       ldz, safe);
  return check_launch("trinv_diag");
}

}  // namespace ifk
