// Single-workgroup kernels on b x b (b <= 64) matrices held in LDS, used by the
// panel factorisation of the streaming fold and by the blocked triangular
// inverse and Cholesky.  Matrices are fp32, padded to 64 x 64 with the
// identity beyond b, row stride SLD.  Dense 64-wide work is blocked: diagonal
// blocks are factored or inverted in registers (the Cholesky leaf redundantly
// in every lane, the inverse leaf one column per lane), off-diagonal blocks
// and products run on fp32 MFMA, so a 64 x 64 Cholesky or inverse needs a
// few workgroup barriers instead of one or more per column.  The second
// CholeskyQR pass factors a Gram matrix close to the identity with MFMA
// fixed-point sweeps instead (sm_chol_near_id, sm_inv_near_id).
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
#include "gemm.h"
#include "kernels.h"

namespace ifk {

constexpr int SB = 64;        // max panel / block width
constexpr int SLD = SB + 1;   // LDS row stride (floats)
constexpr int SNT = 256;
constexpr int TB = 16;        // register tile
constexpr int TRINV_TMP = 2048; // LDS scratch of sm_trinv64 (floats)

__device__ inline float bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// ---------------------------------------------------------------------------
// LDS building blocks (all called by the whole 256-thread workgroup)
// ---------------------------------------------------------------------------

// The two halves of sm_load_pad, for kernels that issue several loads
// before the first is needed: this thread's 16 entries into registers, and
// from registers into LDS (no barrier).
constexpr int PAD_PER = SB * SB / SNT;
__device__ __forceinline__ void ld_pad(float (&v)[PAD_PER], const float* g, int64_t ld, int b,
                                       bool upper, float pad) {
#pragma unroll
  for (int q = 0; q < PAD_PER; ++q) {
    const int e = threadIdx.x + SNT * q;
    const int r = e >> 6, c = e & 63;
    if (r < b && c < b) v[q] = (upper && r > c) ? 0.0f : g[(int64_t)r * ld + c];
    else v[q] = (r == c) ? pad : 0.0f;
  }
}
__device__ __forceinline__ void st_pad(float* S, const float (&v)[PAD_PER]) {
#pragma unroll
  for (int q = 0; q < PAD_PER; ++q) {
    const int e = threadIdx.x + SNT * q;
    S[(e >> 6) * SLD + (e & 63)] = v[q];
  }
}

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
// zeroed on exit).  mode 0: a pivot below tol * (its diagonal on entry, or
// dref[i] for i < b when dref is given) or not finite raises *bad (the
// factorisation continues on a clamped pivot so every thread runs the same
// steps); mode 1: the pivot rule of cholesky_bf16, clamp_min(pivot, 1e-7)
// with a NaN pivot kept NaN.
//
// One wave holds the upper triangle in registers, as three 32 x 32 blocks
// (00, 01, 11) in the fp32 MFMA 32x32 result layout: lane l holds column
// l % 32 of a block, register j its row 8 (j / 4) + 4 (l / 32) + j % 4.  So
// the four rows 4p .. 4p + 3 of a panel sit in four consecutive registers of
// one half of the lanes, across every block of their block row.  Each panel
// is factored on the VALU (its pivots come by readlane, its rows are scaled
// and the later panel rows updated lane = column), then applied to the
// trailing blocks as two rank-2 products on fp32 MFMA, whose operands are the
// panel rows with one row moved to the other half of the lanes
// (v_permlane32_swap) and everything left of the panel's end masked to zero.
// The other waves only meet the two barriers.  (CB is kept for the callers'
// spelling; the panel is four rows.)
//
// With INV, Z (LDS, stride SLD) also receives U^{-1}: the same row operations
// applied to the identity give W = U^{-T} (lower triangular; blocks 00, 10,
// 11 in the same layout, updated by the same pivots, scalings and rank-2
// products), stored transposed.  Wave 1 carries W alongside wave 0: as soon
// as wave 0 has factored a panel it writes the panel's four rows of U (final
// from then on) into A and their pivots' reciprocal square roots into LDS and
// bumps a panel counter; wave 1 takes the row operations' coefficients and
// the rank-2 operands from there, so the inverse costs the factorisation no
// time (the same operations on the same values: W bit for bit as when one
// wave did both).
template <int CB = 32, bool EXACT = false, bool INV = false>
__device__ __forceinline__ void sm_chol64(float* A, float tol, int* bad, int mode,
                                          const float* dref = nullptr, int b = SB,
                                          float* Z = nullptr) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6, l32 = lane & 31, h = lane >> 5;
  __shared__ float dgs[SB];   // reference diagonal of the pivot test
  __shared__ float rsv[SB];   // INV: each pivot's reciprocal square root (wave 0 -> 1)
  __shared__ int panels;      // INV: panels whose rows of U are in A (wave 0 -> 1)
  if (t < SB) dgs[t] = (dref != nullptr && t < b) ? dref[t] : A[t * SLD + t];
  if (INV && t == 0) panels = 0;
  __syncthreads();
  // lane l: row 4p + 2 s2 (l < 32) or the next row (l >= 32) of a panel whose
  // rows sit in the lanes of half hk, from the registers of its two rows
  auto pair = [&](float x0, float x1, int hk) -> float {
    if (hk == 0) {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x1), __float_as_uint(x1),
                                                       false, false);
      return h == 0 ? x0 : __uint_as_float(sw[0]);
    }
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x0), __float_as_uint(x0),
                                                     false, false);
    return h == 0 ? __uint_as_float(sw[1]) : x1;
  };
  if (wave == 0) {
    f32x16 b00, b01, b11;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = (j >> 2) * 8 + h * 4 + (j & 3);
      b00[j] = (r <= l32) ? A[r * SLD + l32] : 0.0f;
      b01[j] = A[r * SLD + 32 + l32];
      b11[j] = (r <= l32) ? A[(32 + r) * SLD + 32 + l32] : 0.0f;
    }
    int flag = 0;
    const float dgv = dgs[lane];            // the reference diagonal, lane k holding k's
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const int K = p >> 3;                 // block row of the panel
      const int hk = p & 1;                 // the half of the lanes holding its rows
      const int jb = ((p & 7) >> 1) * 4;    // and their registers jb .. jb + 3
      const bool mine = h == hk;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int k = 4 * p + q, kk = k & 31, reg = jb + q;
        const float piv = bcast(K == 0 ? b00[reg] : b11[reg], kk + 32 * hk);
        float rs, dg;
        if (mode == 0) {
          if (!(piv > tol * bcast(dgv, k)) || !isfinite(piv)) flag = 1;
          const float pv = fmaxf(piv, 1e-30f);
          if (EXACT) {
            // correctly rounded: a first pass whose second pass cannot carry
            // a sub-ulp correction must not add a biased one (v_rsq_f32's
            // error is systematic, and a stream of folds compounds it)
            dg = sqrtf(pv);
            rs = 1.0f / dg;
          } else {
            rs = __builtin_amdgcn_rsqf(pv);
            dg = pv * rs;
          }
        } else {
          // clamp_min(1e-7) of cholesky_bf16 (bf16_linalg.py:258): a NaN
          // pivot stays NaN (fmaxf would return the bound)
          dg = sqrtf((piv >= 1e-7f || piv != piv) ? piv : 1e-7f);
          rs = 1.0f / dg;
        }
        if (INV && lane == 0) rsv[k] = rs;
        // row k of U: its half's lanes of every block in block row K
        if (K == 0) {
          b00[reg] = mine ? ((l32 == kk) ? dg : b00[reg] * rs) : b00[reg];
          b01[reg] = mine ? b01[reg] * rs : b01[reg];
        } else {
          b11[reg] = mine ? ((l32 == kk) ? dg : b11[reg] * rs) : b11[reg];
        }
        // the panel's later rows
#pragma unroll
        for (int q2 = q + 1; q2 < 4; ++q2) {
          const int r2 = jb + q2;
          const float c = bcast(K == 0 ? b00[reg] : b11[reg], ((4 * p + q2) & 31) + 32 * hk);
          if (K == 0) {
            b00[r2] = mine ? fmaf(-c, b00[reg], b00[r2]) : b00[r2];
            b01[r2] = mine ? fmaf(-c, b01[reg], b01[r2]) : b01[r2];
          } else {
            b11[r2] = mine ? fmaf(-c, b11[reg], b11[r2]) : b11[r2];
          }
        }
      }
      if (INV) {
        // the panel's rows of U are final: into A (zero left of the
        // diagonal) for wave 1
        if (mine) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int k = 4 * p + q, reg = jb + q;
            if (K == 0) {
              A[k * SLD + l32] = (k <= l32) ? b00[reg] : 0.0f;
              A[k * SLD + 32 + l32] = b01[reg];
            } else {
              A[k * SLD + l32] = 0.0f;
              A[k * SLD + 32 + l32] = (k - 32 <= l32) ? b11[reg] : 0.0f;
            }
          }
        }
      }
      if (p == 15) {
        if (INV && lane == 0)
          __hip_atomic_store(&panels, 16, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        break;
      }
      // the panel applied to rows and columns from pend on: two rank-2 products
      const int pend = 4 * p + 4;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int r0 = jb + 2 * s2, r1 = r0 + 1;
        auto opnd = [&](float x0, float x1, int colbase) -> float {
          const float v = pair(x0, x1, hk);
          return (colbase + l32 >= pend) ? v : 0.0f;
        };
        if (K == 0) {
          const float u0 = opnd(b00[r0], b00[r1], 0), u1 = opnd(b01[r0], b01[r1], 32);
          if (pend < 32) b00 = __builtin_amdgcn_mfma_f32_32x32x2f32(-u0, u0, b00, 0, 0, 0);
          b01 = __builtin_amdgcn_mfma_f32_32x32x2f32(-u0, u1, b01, 0, 0, 0);
          b11 = __builtin_amdgcn_mfma_f32_32x32x2f32(-u1, u1, b11, 0, 0, 0);
        } else {
          const float u1 = opnd(b11[r0], b11[r1], 32);
          b11 = __builtin_amdgcn_mfma_f32_32x32x2f32(-u1, u1, b11, 0, 0, 0);
        }
      }
      // the count behind the rank-2 products: the row writes have landed by
      // now, so its wait for them costs nothing
      if (INV && lane == 0)
        __hip_atomic_store(&panels, p + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (!INV) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int r = (j >> 2) * 8 + h * 4 + (j & 3);
        A[r * SLD + l32] = (r <= l32) ? b00[j] : 0.0f;
        A[r * SLD + 32 + l32] = b01[j];
        A[(32 + r) * SLD + l32] = 0.0f;
        A[(32 + r) * SLD + 32 + l32] = (r <= l32) ? b11[j] : 0.0f;
      }
    }
    if (flag && bad) *bad = 1;
  } else if (INV && wave == 1) {
    f32x16 w00, w10, w11;   // W = U^{-T}, from the identity
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = (j >> 2) * 8 + h * 4 + (j & 3);
      w00[j] = (r == l32) ? 1.0f : 0.0f;
      w10[j] = 0.0f;
      w11[j] = (r == l32) ? 1.0f : 0.0f;
    }
    bool late = false;
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const int K = p >> 3, hk = p & 1, jb = ((p & 7) >> 1) * 4;
      const bool mine = h == hk;
      // wave 0 runs ahead and never waits for this wave, so the wait ends;
      // the bound only keeps a broken count from spinning forever
      for (int it = 0; __hip_atomic_load(&panels, __ATOMIC_ACQUIRE,
                                         __HIP_MEMORY_SCOPE_WORKGROUP) < p + 1; ++it) {
        if (it > (1 << 22)) {
          late = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int k = 4 * p + q, reg = jb + q;
        const float rs = rsv[k];
        if (K == 0) {
          w00[reg] = mine ? w00[reg] * rs : w00[reg];
        } else {
          w10[reg] = mine ? w10[reg] * rs : w10[reg];
          w11[reg] = mine ? w11[reg] * rs : w11[reg];
        }
#pragma unroll
        for (int q2 = q + 1; q2 < 4; ++q2) {
          const int r2 = jb + q2;
          const float c = A[k * SLD + 4 * p + q2];   // U[k][4p + q2]
          if (K == 0) {
            w00[r2] = mine ? fmaf(-c, w00[reg], w00[r2]) : w00[r2];
          } else {
            w10[r2] = mine ? fmaf(-c, w10[reg], w10[r2]) : w10[r2];
            w11[r2] = mine ? fmaf(-c, w11[reg], w11[r2]) : w11[r2];
          }
        }
      }
      if (p == 15) break;
      const int pend = 4 * p + 4;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int r0 = jb + 2 * s2, r1 = r0 + 1;
        // the rank-2 operands wave 0 uses, from the rows of U in A
        const int row = 4 * p + 2 * s2 + h;
        const float u1 = (32 + l32 >= pend) ? A[row * SLD + 32 + l32] : 0.0f;
        if (K == 0) {
          const float u0 = (l32 >= pend) ? A[row * SLD + l32] : 0.0f;
          const float v0 = pair(w00[r0], w00[r1], hk);
          if (pend < 32) w00 = __builtin_amdgcn_mfma_f32_32x32x2f32(-u0, v0, w00, 0, 0, 0);
          w10 = __builtin_amdgcn_mfma_f32_32x32x2f32(-u1, v0, w10, 0, 0, 0);
        } else {
          const float v0 = pair(w10[r0], w10[r1], hk), v1 = pair(w11[r0], w11[r1], hk);
          w10 = __builtin_amdgcn_mfma_f32_32x32x2f32(-u1, v0, w10, 0, 0, 0);
          w11 = __builtin_amdgcn_mfma_f32_32x32x2f32(-u1, v1, w11, 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = (j >> 2) * 8 + h * 4 + (j & 3);
      // Z = W^T: W's element (row, col) goes to Z[col][row]
      Z[l32 * SLD + r] = (r >= l32) ? w00[j] : 0.0f;
      Z[l32 * SLD + 32 + r] = w10[j];
      Z[(32 + l32) * SLD + r] = 0.0f;
      Z[(32 + l32) * SLD + 32 + r] = (r >= l32) ? w11[j] : 0.0f;
    }
    if (late && bad) *bad = 1;
  }
  __syncthreads();
}

// Z = U^{-1} for a padded 64 x 64 upper-triangular U (Z strict lower = 0).
// With safe set, diagonal divisors follow safe_divisor.  Wave w inverts the
// 16 x 16 diagonal block w (lane j holds
// column j; back substitution with the row of U read from LDS as a broadcast),
// then the off-diagonal blocks follow by recursive doubling,
// Z_12 = -Z_11 U_12 Z_22, at 16 and 32 on fp32 MFMA (32 x 32 tiles, zero
// padded at level 16).  Tmp: LDS scratch of TRINV_TMP floats.
__device__ __forceinline__ void sm_trinv64(const float* U, float* Z, float* Tmp,
                                             bool safe = false) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  for (int e = t; e < SB * SB; e += SNT) Z[(e >> 6) * SLD + (e & 63)] = 0.0f;
  __syncthreads();
  {
    const int o = wave * TB;
    float z[TB], rd[TB];
#pragma unroll
    for (int i = 0; i < TB; ++i) {
      const float dv = U[(o + i) * SLD + o + i];
      rd[i] = 1.0f / (safe ? safe_divisor(dv) : dv);
    }
#pragma unroll
    for (int i = TB - 1; i >= 0; --i) {
      float s = (i == lane) ? 1.0f : 0.0f;
#pragma unroll
      for (int k = i + 1; k < TB; ++k) s = fmaf(-U[(o + i) * SLD + o + k], z[k], s);
      z[i] = s * rd[i];
    }
    if (lane < TB) {
#pragma unroll
      for (int i = 0; i < TB; ++i) Z[(o + i) * SLD + o + lane] = z[i];
    }
  }
  __syncthreads();
  // level 16: for pair pr (waves 0, 1), blocks (o0, o1) = (32 pr, 32 pr + 16):
  // Tmp_pr = U[o0:o0+16, o1:o1+16] Z[o1.., o1..], then Z[o0.., o1..] = -Z[o0.., o0..] Tmp_pr.
  // A 32 x 32 MFMA tile with rows / columns >= 16 and k >= 16 zero.
  if (wave < 2) {
    const int o0 = 32 * wave, o1 = o0 + 16;
    f32x16 d;
#pragma unroll
    for (int i = 0; i < 16; ++i) d[i] = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < 8; ++s2) {
      const int k = 8 * h + s2;    // 0..15
      const float a = (l32 < 16) ? U[(o0 + l32) * SLD + o1 + k] : 0.0f;
      const float b = (l32 < 16) ? Z[(o1 + k) * SLD + o1 + l32] : 0.0f;
      d = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, d, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = (i >> 2) * 8 + h * 4 + (i & 3);
      if (row < 16 && l32 < 16) Tmp[wave * 256 + row * 16 + l32] = d[i];
    }
  }
  __syncthreads();
  if (wave < 2) {
    const int o0 = 32 * wave, o1 = o0 + 16;
    f32x16 d;
#pragma unroll
    for (int i = 0; i < 16; ++i) d[i] = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < 8; ++s2) {
      const int k = 8 * h + s2;
      const float a = (l32 < 16) ? Z[(o0 + l32) * SLD + o0 + k] : 0.0f;
      const float b = (l32 < 16) ? Tmp[wave * 256 + k * 16 + l32] : 0.0f;
      d = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, d, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = (i >> 2) * 8 + h * 4 + (i & 3);
      if (row < 16 && l32 < 16) Z[(o0 + row) * SLD + o1 + l32] = -d[i];
    }
  }
  __syncthreads();
  // level 32: Tmp = U[0:32, 32:64] Z[32:64, 32:64], Z[0:32, 32:64] = -Z[0:32, 0:32] Tmp,
  // one 32 x 32 tile, K = 32 split over two waves (partial sums added in LDS).
  if (wave < 2) {
    f32x16 d;
#pragma unroll
    for (int i = 0; i < 16; ++i) d[i] = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < 8; ++s2) {
      const int k = 16 * wave + 8 * h + s2;   // 0..31
      d = __builtin_amdgcn_mfma_f32_32x32x2f32(U[l32 * SLD + 32 + k], Z[(32 + k) * SLD + 32 + l32],
                                               d, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = (i >> 2) * 8 + h * 4 + (i & 3);
      Tmp[wave * 1024 + row * 32 + l32] = d[i];
    }
  }
  __syncthreads();
  f32x16 d2;
#pragma unroll
  for (int i = 0; i < 16; ++i) d2[i] = 0.0f;
  if (wave < 2) {
#pragma unroll
    for (int s2 = 0; s2 < 8; ++s2) {
      const int k = 16 * wave + 8 * h + s2;
      const float b = Tmp[k * 32 + l32] + Tmp[1024 + k * 32 + l32];
      d2 = __builtin_amdgcn_mfma_f32_32x32x2f32(Z[l32 * SLD + k], b, d2, 0, 0, 0);
    }
  }
  __syncthreads();   // every read of Tmp precedes the partial sum written below
  if (wave == 1) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = (i >> 2) * 8 + h * 4 + (i & 3);
      Tmp[row * 32 + l32] = d2[i];
    }
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = (i >> 2) * 8 + h * 4 + (i & 3);
      Z[row * SLD + 32 + l32] = -(d2[i] + Tmp[row * 32 + l32]);
    }
  }
  __syncthreads();
}

// max over the padded 64 x 64 matrix of |A_ij - d * delta_ij|, returned to
// every thread.  red: LDS scratch of 4 floats.
__device__ __forceinline__ float sm_maxabs(const float* A, float d, float* red) {
  const int t = threadIdx.x;
  float m = 0.0f;
#pragma unroll
  for (int q = 0; q < SB * SB / SNT; ++q) {
    const int e = t + SNT * q, i = e >> 6, j = e & 63;
    m = fmaxf(m, fabsf(A[i * SLD + j] - (i == j ? d : 0.0f)));
  }
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  __syncthreads();   // red may still be read by a previous call
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Upper Cholesky factor of a matrix close to the identity, A = I + E with E
// small (the Gram matrix of the second CholeskyQR pass).  With U = I + F and
// F upper triangular, U^T U = A is the fixed point
//   F = up(E - F^T F),  up(X) = strict upper part of X + diag(X) / 2,
// which contracts at a rate of about 2 ||F|| from F_0 = up(E); each sweep is
// one 64 x 64 MFMA product.  On success A holds U (strict lower part zero),
// F holds U - I unrounded, and the function returns true; when the sweeps
// have not settled below 2^-26 after maxit (E not small enough) A is left
// unchanged and it returns false.  With one = 0, A holds E itself on entry
// (for callers that form E without rounding I + E).  F, P: LDS scratch
// (padded 64 x 64), red: 4 floats.
__device__ __forceinline__ bool sm_chol_near_id(float* A, float* F, float* P, float* red,
                                                int maxit, float one = 1.0f) {
  const int t = threadIdx.x;
  for (int e = t; e < SB * SB; e += SNT) {
    const int i = e >> 6, j = e & 63;
    const float x = A[i * SLD + j] - (i == j ? one : 0.0f);
    F[i * SLD + j] = (i < j) ? x : (i == j ? 0.5f * x : 0.0f);
  }
  __syncthreads();
  bool done = false;
  for (int it = 0; it < maxit && !done; ++it) {
    sm_gemm64<true, false>(F, F, P, 1.0f, false);      // P = F^T F
    float dmax = 0.0f;
#pragma unroll
    for (int q = 0; q < SB * SB / SNT; ++q) {
      const int e = t + SNT * q, i = e >> 6, j = e & 63;
      if (i <= j) {
        const float x = A[i * SLD + j] - (i == j ? one : 0.0f) - P[i * SLD + j];
        const float f = (i < j) ? x : 0.5f * x;
        dmax = fmaxf(dmax, fabsf(f - F[i * SLD + j]));
        F[i * SLD + j] = f;
      }
    }
    for (int o = 32; o > 0; o >>= 1) dmax = fmaxf(dmax, __shfl_xor(dmax, o));
    __syncthreads();
    if ((t & 63) == 0) red[t >> 6] = dmax;
    __syncthreads();
    done = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) <= 1.4901161e-8f;
  }
  if (!done) return false;
  for (int e = t; e < SB * SB; e += SNT) {
    const int i = e >> 6, j = e & 63;
    A[i * SLD + j] = (i <= j) ? F[i * SLD + j] + (i == j ? 1.0f : 0.0f) : 0.0f;
  }
  __syncthreads();
  return true;
}

// Z = U^{-1} for U = I + F with F upper triangular and small (padded 64 x 64):
// the Neumann series I - F + F^2 - ..., one MFMA product per term, stopped
// once a term is below 2^-30 in every entry.  Returns false (Z undefined)
// when maxit terms do not get there.  Tm, P: LDS scratch, red: 4 floats.
__device__ __forceinline__ bool sm_inv_near_id(const float* U, float* Z, float* Tm, float* P,
                                               float* red, int maxit) {
  const int t = threadIdx.x;
  // F = U - I into P, Z = I - F, Tm = -F (the current term)
  for (int e = t; e < SB * SB; e += SNT) {
    const int i = e >> 6, j = e & 63;
    const float f = U[i * SLD + j] - (i == j ? 1.0f : 0.0f);
    P[i * SLD + j] = f;
    Tm[i * SLD + j] = -f;
    Z[i * SLD + j] = (i == j ? 1.0f : 0.0f) - f;
  }
  __syncthreads();
  for (int it = 0; it < maxit; ++it) {
    if (sm_maxabs(Tm, 0.0f, red) <= 9.3132257e-10f) return true;
    sm_gemm64<false, false>(Tm, P, Tm, -1.0f, false);   // term <- -term F
    for (int e = t; e < SB * SB; e += SNT) {
      const int i = e >> 6, j = e & 63;
      Z[i * SLD + j] += Tm[i * SLD + j];
    }
    __syncthreads();
  }
  return sm_maxabs(Tm, 0.0f, red) <= 9.3132257e-10f;
}

// ---------------------------------------------------------------------------
// Panel kernels
// ---------------------------------------------------------------------------

// CholeskyQR pass 1.  In: G = X_p^T X_p (64 x 64, ld 64), P_top (in R at ldr).
// Out: U1 (Cholesky factor of P^T P), M1 = U1^{-1}, Q1 = P_top M1 (b x b,
// ld b); *flag = 1 when a pivot falls below tol times its diagonal (the
// panel then goes to the Householder fallback), else 0.
//
// P^T P = X_p^T X_p + P_top^T P_top is summed in fp64 before its one
// rounding to fp32: along a stream the running factor's block P_top grows
// with the rows folded so far and dominates the sum, and the fp32 rounding of
// its 64-term products, repeated fold after fold, would add up (200 folds of
// 4096 rows into a 512-column factor: 2e-6 relative Gram error where fp32
// Householder QR keeps 1.4e-7; with the sum in fp64 the fold keeps the
// latter).
__global__ __launch_bounds__(SNT) void panel_hr_a_kernel(const float* G,
                                                          const float* Ptop, int64_t ldr, int b,
                                                          float tol, float* U1, float* M1,
                                                          float* Q1, int* flag) {
  __shared__ float sG[SB * SLD];
  __shared__ float sP[SB * SLD];
  __shared__ float sM[SB * SLD];
  __shared__ float sT[TRINV_TMP];
  __shared__ double sG64[SB * SB];
  __shared__ int bad;
  const int t = threadIdx.x;
  if (t == 0) bad = 0;
  {
    float vg[PAD_PER], vp[PAD_PER];   // both loads in flight together
    ld_pad(vg, G, SB, b, false, 1.0f);
    ld_pad(vp, Ptop, ldr, b, true, 0.0f);
    st_pad(sG, vg);
    st_pad(sP, vp);
    __syncthreads();
  }
  // sG64 = X_p^T X_p + P_top^T P_top (P_top upper triangular: k <= min(i, j));
  // beyond b the identity of the pad
  for (int e = t; e < SB * SB; e += SNT) {
    const int i = e >> 6, j = e & 63;
    double v = (double)sG[i * SLD + j];
    const int km = min(i, j);
    for (int k = 0; k <= km; ++k) v += (double)sP[k * SLD + i] * (double)sP[k * SLD + j];
    sG64[e] = v;
  }
  __syncthreads();
  for (int e = t; e < SB * SB; e += SNT) sG[(e >> 6) * SLD + (e & 63)] = (float)sG64[e];
  __syncthreads();
  sm_chol64<32, true>(sG, tol, &bad, 0);           // sG = U1
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
  __shared__ float sTmp[TRINV_TMP];
  __shared__ float sgn[SB];
  __shared__ int bad;
  const int t = threadIdx.x;
  const int role = blockIdx.x;   // 0: R_new and N; 1 + cb: block cb of the rest
  const int cb = role - 1;
  const int c0 = cb * SB;
  const int w = role > 0 ? ((nr - c0) < SB ? (nr - c0) : SB) : 0;
  float* Rrest = R + b;
  if (t == 0) bad = 0;
  // every global operand of this workgroup in flight at once: G2, Q1, and
  // U1 (role 0) or this block's Q2^T C and R_rest (the others)
  float vG[PAD_PER], vQ[PAD_PER], vX[PAD_PER], vR[PAD_PER];
  ld_pad(vG, G, SB, b, false, 1.0f);
  ld_pad(vQ, Q1, b, b, true, 0.0f);
  if (role == 0) {
    ld_pad(vX, U1, b, b, true, 1.0f);
  } else {
    ld_pad(vX, G + (size_t)(1 + cb) * SB * SB, SB, SB, false, 1.0f);
#pragma unroll
    for (int q = 0; q < PAD_PER; ++q) {
      const int e = t + SNT * q, i = e >> 6, j = e & 63;
      vR[q] = (i < b && j < w) ? Rrest[(int64_t)i * ldr + c0 + j] : 0.0f;
    }
  }
  const bool flagged = (*flag != 0);
  bool near = false;
  float vF[PAD_PER];
  st_pad(sG, vG);
  __syncthreads();
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
    st_pad(sQ, vQ);
    __syncthreads();
    // after the first pass G2 = Q^T Q is I + E with E small.  E is formed
    // without rounding I + E to fp32 -- near 1 that rounding is as large as
    // E, and along a stream the lost correction adds up fold after fold --
    // from D = Q1 - I (exact):  E = Q2^T Q2 + D + D^T + D^T D  (zero in the
    // pad, where sG holds the identity).
    for (int e = t; e < SB * SB; e += SNT) {
      const int i = e >> 6, j = e & 63;
      sM[i * SLD + j] = (i < b && j < b) ? sQ[i * SLD + j] - (i == j ? 1.0f : 0.0f) : 0.0f;
    }
    __syncthreads();
    for (int e = t; e < SB * SB; e += SNT) {
      const int i = e >> 6, j = e & 63;
      const float g = sG[i * SLD + j];
      sG[i * SLD + j] = (i < b && j < b) ? g + sM[i * SLD + j] + sM[j * SLD + i] : 0.0f;
    }
    __syncthreads();
    sm_gemm64<true, false>(sM, sM, sG, 1.0f, true);  // sG = E
    // a few MFMA sweeps give U2 (and F = U2 - I) and M2; the general
    // Cholesky / inverse of I + E are the fallback
    near = sm_chol_near_id(sG, sX, sM, sgn, 8, 0.0f);   // sG = U2
    if (near) {
      // F = U2 - I exactly as the sweeps left it: U2 itself, rounded next to
      // 1, drops corrections below half an ulp of 1
#pragma unroll
      for (int q = 0; q < PAD_PER; ++q) {
        const int e = t + SNT * q;
        vF[q] = sX[(e >> 6) * SLD + (e & 63)];
      }
    } else {
      for (int j = t; j < SB; j += SNT) sG[j * SLD + j] += 1.0f;   // I + E
      __syncthreads();
      sm_chol64(sG, 0.25f, &bad, 0);
    }
    if (!(near && sm_inv_near_id(sG, sM, sX, sN, sgn, 8)))   // sM = M2
      sm_trinv64(sG, sM, sTmp);
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
    st_pad(sM, vX);
    const float nan = __int_as_float(0x7fc00000);
    if (near) {
      // R_new = S (U1 + F U1), with U2 = I + F
      st_pad(sG, vF);
      __syncthreads();
      sm_gemm64<false, false>(sG, sM, sX, 1.0f, false);  // sX = F U1
      for (int e = t; e < b * b; e += SNT) {
        const int i = e / b, j = e - i * b;
        R[(int64_t)i * ldr + j] =
            !ok ? nan : ((i <= j) ? sgn[i] * (sM[i * SLD + j] + sX[i * SLD + j]) : 0.0f);
      }
      return;
    }
    __syncthreads();
    sm_gemm64<false, false>(sG, sM, sM, 1.0f, false);  // sM = U2 U1
    for (int e = t; e < b * b; e += SNT) {           // R_new = S U2 U1
      const int i = e / b, j = e - i * b;
      R[(int64_t)i * ldr + j] = !ok ? nan : ((i <= j) ? sgn[i] * sM[i * SLD + j] : 0.0f);
    }
    return;
  }
  // block cb of the rest: columns [b + c0, b + c0 + w) of R's block row
  st_pad(sG, vX);                                      // Q2^T C block
  __syncthreads();
  sm_gemm64<true, false>(sQ, sG, sM, 1.0f, false);     // sM = W = NT^T (Q2^T C)
  st_pad(sG, vR);                                      // R_rest
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
// rule, bf16_linalg.py:258-260): U_jj = sqrt(clamp_min(A_jj - sum_k U_kj^2, 1e-7)),
// a NaN pivot kept NaN.
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

// ---------------------------------------------------------------------------
// Blocked upper Cholesky of an n x n fp32 matrix (n <= CHOLB_MAX) held in
// global memory, for the CholeskyQR of a whole outer block of the fold.
// Right-looking over 64-column steps, one launch per step:
//   cholb_first:   dref = diag(A) (the reference of the pivot test), then
//                  U_00 = chol(A_00) and Z_0 = U_00^{-1}
//   cholb_step k:  workgroup (i, j), k < i <= j: U_ki = Z_k^T A_ki and
//                  U_kj = Z_k^T A_kj (each workgroup forms the two blocks it
//                  needs), A_ij -= U_ki^T U_kj; workgroup (j, j) stores U_kj;
//                  workgroup (k+1, k+1) goes on to factor its updated block,
//                  U_{k+1,k+1} and Z_{k+1}, which the next step reads.
// A launch reads block row k of A and writes only blocks (i, j) with i > k,
// so its workgroups never race.  U (ld ldu) receives the blocks on and above
// the diagonal (the ones below are not written); Zd holds the 64 x 64
// inverses of the diagonal blocks (identity beyond n).  A pivot below tol *
// dref[i] or not finite sets *flag (the factorisation goes on with clamped
// pivots, so every launch still runs the same steps).
// ---------------------------------------------------------------------------
constexpr int CHOLB_MAX = 16 * SB;

// rows x cols block (row stride ld) into registers as a padded 64 x 64 tile:
// outside the block the tile is pad * I
__device__ __forceinline__ void ld_blk(float (&v)[PAD_PER], const float* g, int64_t ld, int rows,
                                       int cols, float pad) {
#pragma unroll
  for (int q = 0; q < PAD_PER; ++q) {
    const int e = threadIdx.x + SNT * q;
    const int r = e >> 6, c = e & 63;
    v[q] = (r < rows && c < cols) ? g[(int64_t)r * ld + c] : (r == c ? pad : 0.0f);
  }
}

__device__ __forceinline__ void st_blk(const float* S, float* g, int64_t ld, int rows, int cols) {
  for (int e = threadIdx.x; e < SB * SB; e += SNT) {
    const int r = e >> 6, c = e & 63;
    if (r < rows && c < cols) g[(int64_t)r * ld + c] = S[r * SLD + c];
  }
}

__global__ __launch_bounds__(SNT) void cholb_first_kernel(const float* A, int64_t lda, int n,
                                                          float* U, int64_t ldu, float* Zd,
                                                          float* dref, float tol, int* flag,
                                                          float* Mo, int64_t ldm, int dref_in,
                                                          CholbStrides bs) {
  // batch entry blockIdx.y
  {
    const int64_t b = blockIdx.y;
    A += b * bs.a; U += b * bs.u; Zd += b * bs.zd; dref += b * bs.dref; flag += b * bs.flag;
    if (Mo) Mo += b * bs.m;
  }
  __shared__ float sC[SB * SLD];
  __shared__ float sZ[SB * SLD];
  __shared__ int bad;
  const int t = threadIdx.x;
  const int b0 = n < SB ? n : SB;
  if (t == 0) bad = 0;
  if (!dref_in)
    for (int e = t; e < n; e += SNT) dref[e] = A[(int64_t)e * lda + e];
  float v[PAD_PER];
  ld_blk(v, A, lda, b0, b0, 1.0f);
  st_pad(sC, v);
  __syncthreads();
  // block 0: its diagonal on entry is A's (or the given reference); its
  // inverse alongside
  sm_chol64<32, false, true>(sC, tol, &bad, 0, dref_in ? dref : nullptr, b0, sZ);
  st_blk(sC, U, ldu, b0, b0);
  for (int e = t; e < SB * SB; e += SNT) {
    const int r = e >> 6, c = e & 63;
    Zd[e] = sZ[r * SLD + c];
    if (Mo && r < b0 && c < b0) Mo[(int64_t)r * ldm + c] = sZ[r * SLD + c];
  }
  if (t == 0 && bad) *flag = 1;
}

__global__ __launch_bounds__(SNT) void cholb_step_kernel(float* A, int64_t lda, int n, float* U,
                                                         int64_t ldu, float* Zd,
                                                         const float* dref, float tol, int* flag,
                                                         int k, float* Mo, int64_t ldm,
                                                         CholbStrides bs) {
  {
    const int64_t b = blockIdx.y;
    A += b * bs.a; U += b * bs.u; Zd += b * bs.zd; dref += b * bs.dref; flag += b * bs.flag;
    if (Mo) Mo += b * bs.m;
  }
  __shared__ float sZ[SB * SLD];
  __shared__ float sA[SB * SLD];
  __shared__ float sB[SB * SLD];
  __shared__ float sC[SB * SLD];
  __shared__ int bad;
  const int t = threadIdx.x;
  const int nb = (n + SB - 1) / SB;
  const int nupd = (nb - 1 - k) * (nb - k) / 2;
  if ((int)blockIdx.x >= nupd) {
    // M = U^{-1} by column blocks: M_kk = Z_k and, for i < k,
    //   M_ik = -(sum_{l = i}^{k-1} M_il U_lk) Z_k.
    // The sum is built up across launches in M_ik's own place: launch k adds
    // the terms l = k - 1 of the columns kk > k (storing, not adding, the
    // first term l = i), and finishes column k with its own l = k - 1 term,
    // so no workgroup multiplies more than two blocks.  Every block read
    // here was finished by an earlier launch.
    const int idx = (int)blockIdx.x - nupd;
    float va[PAD_PER], vb[PAD_PER], vc[PAD_PER];
    if (idx > k) {
      const int w = nb - 1 - k, a = idx - (k + 1);
      const int i = a / w, kk = k + 1 + a % w;   // i < k < kk < nb
      const int bkk = (n - SB * kk) < SB ? (n - SB * kk) : SB;
      const bool first = (i == k - 1);
      ld_blk(va, Mo + (int64_t)SB * i * ldm + SB * (k - 1), ldm, SB, SB, 0.0f);
      ld_blk(vb, U + (int64_t)SB * (k - 1) * ldu + SB * kk, ldu, SB, bkk, 0.0f);
      if (first) {
#pragma unroll
        for (int q = 0; q < PAD_PER; ++q) vc[q] = 0.0f;
      } else {
        ld_blk(vc, Mo + (int64_t)SB * i * ldm + SB * kk, ldm, SB, bkk, 0.0f);
      }
      st_pad(sA, va);
      st_pad(sB, vb);
      st_pad(sC, vc);
      __syncthreads();
      sm_gemm64<false, false>(sA, sB, sC, 1.0f, true);
      st_blk(sC, Mo + (int64_t)SB * i * ldm + SB * kk, ldm, SB, bkk);
      return;
    }
    const int i = idx;
    const int bk = (n - SB * k) < SB ? (n - SB * k) : SB;
    const float* Zk = Zd + (size_t)k * SB * SB;
    if (i == k) {
      for (int e = t; e < SB * SB; e += SNT) {
        const int r = e >> 6, c = e & 63;
        if (r < bk && c < bk) Mo[(int64_t)(SB * k + r) * ldm + SB * k + c] = Zk[e];
      }
      return;
    }
    float vz[PAD_PER];
    ld_blk(va, Mo + (int64_t)SB * i * ldm + SB * (k - 1), ldm, SB, SB, 0.0f);
    ld_blk(vb, U + (int64_t)SB * (k - 1) * ldu + SB * k, ldu, SB, bk, 0.0f);
    if (i == k - 1) {
#pragma unroll
      for (int q = 0; q < PAD_PER; ++q) vc[q] = 0.0f;
    } else {
      ld_blk(vc, Mo + (int64_t)SB * i * ldm + SB * k, ldm, SB, bk, 0.0f);
    }
#pragma unroll
    for (int q = 0; q < PAD_PER; ++q) vz[q] = Zk[t + SNT * q];
    st_pad(sA, va);
    st_pad(sB, vb);
    st_pad(sC, vc);
    st_pad(sZ, vz);
    __syncthreads();
    sm_gemm64<false, false>(sA, sB, sC, 1.0f, true);     // C = P_ik + M_i,k-1 U_k-1,k
    sm_gemm64<false, false>(sC, sZ, sA, -1.0f, false);   // M_ik = -C Z_k
    st_blk(sA, Mo + (int64_t)SB * i * ldm + SB * k, ldm, SB, bk);
    return;
  }
  // workgroup -> (i, j), k < i <= j < nb, row by row
  int idx = blockIdx.x, i = k + 1;
  while (idx >= nb - i) {
    idx -= nb - i;
    ++i;
  }
  const int j = i + idx;
  const int bi = (n - SB * i) < SB ? (n - SB * i) : SB;
  const int bj = (n - SB * j) < SB ? (n - SB * j) : SB;
  const bool diag = (i == j);
  if (t == 0) bad = 0;
  const float* Ak = A + (int64_t)SB * k * lda;   // block row k (full: k < nb - 1)
  float vz[PAD_PER], va[PAD_PER], vb[PAD_PER], vc[PAD_PER];
#pragma unroll
  for (int q = 0; q < PAD_PER; ++q) vz[q] = Zd[(size_t)k * SB * SB + t + SNT * q];
  ld_blk(va, Ak + SB * i, lda, SB, bi, 0.0f);
  if (!diag) ld_blk(vb, Ak + SB * j, lda, SB, bj, 0.0f);
  ld_blk(vc, A + (int64_t)SB * i * lda + SB * j, lda, bi, bj, diag ? 1.0f : 0.0f);
  st_pad(sZ, vz);
  st_pad(sA, va);
  if (!diag) st_pad(sB, vb);
  st_pad(sC, vc);
  __syncthreads();
  sm_gemm64<true, false>(sZ, sA, sA, 1.0f, false);                // U_ki
  if (!diag) sm_gemm64<true, false>(sZ, sB, sB, 1.0f, false);     // U_kj
  if (diag) st_blk(sA, U + (int64_t)SB * k * ldu + SB * j, ldu, SB, bj);
  sm_gemm64<true, false>(sA, diag ? sA : sB, sC, -1.0f, true);    // A_ij -= U_ki^T U_kj
  if (diag && i == k + 1) {
    sm_chol64<32, false, true>(sC, tol, &bad, 0, dref + SB * i, bi, sZ);
    st_blk(sC, U + (int64_t)SB * i * ldu + SB * i, ldu, bi, bi);
    for (int e = t; e < SB * SB; e += SNT)
      Zd[(size_t)i * SB * SB + e] = sZ[(e >> 6) * SLD + (e & 63)];
    if (t == 0 && bad) *flag = 1;
  } else {
    st_blk(sC, A + (int64_t)SB * i * lda + SB * j, lda, bi, bj);
  }
}

// hi = RNE bf16(src), lo = RNE bf16(src - hi) (rows x cols, fp32 src), written
// transposed (hi[c][r]) when trans is set
__global__ void split_bf16_kernel(const float* src, int64_t lds, int64_t rows, int64_t cols,
                                  bf16_t* hi, bf16_t* lo, int64_t ldo, int trans) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / cols, c = e % cols;
    const float x = src[r * lds + c];
    const bf16_t h = f32_to_bf16(x);
    const int64_t o = trans ? c * ldo + r : r * ldo + c;
    hi[o] = h;
    lo[o] = f32_to_bf16(x - bf16_to_f32(h));
  }
}

// *status = 2 when *flag is set (a single thread)
__global__ void status_merge_kernel(int* status, const int* flag) {
  if (threadIdx.x == 0 && blockIdx.x == 0 && *flag != 0) *status = 2;
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
                                                         int nb, float* Z, int64_t ldz, int safe,
                                                         bf16_t* Zb, bf16_t* ZTb, int64_t ldb) {
  __shared__ float sU[SB * SLD];
  __shared__ float sZ[SB * SLD];
  __shared__ float sT[TRINV_TMP];
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
    const float z = sZ[r * SLD + c];
    Z[(k0 + r) * ldz + k0 + c] = z;
    if (Zb) Zb[(k0 + r) * ldb + k0 + c] = f32_to_bf16(z);
    if (ZTb) ZTb[(k0 + c) * ldb + k0 + r] = f32_to_bf16(z);
  }
}

// ---------------------------------------------------------------------------
// Diagonal 128 x 128 blocks of a blocked triangular inverse, one workgroup
// per block (the last may be ragged): the two 64-blocks in LDS, then
// Z12 = -Z11 (R12 Z22), so the doubling levels of trinv_core start at 128.
// With ut, R holds a reflector Gram matrix G and the inverted matrix is its
// UT transform striu(G) + diag(1 + diag G) / 2.
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ void load_blk(float* S, const void* R, int64_t ldr, int64_t r0,
                                         int64_t c0, int rows, int cols, bool diag, int ut) {
  float v[SB * SB / SNT];
#pragma unroll
  for (int q = 0; q < SB * SB / SNT; ++q) {
    const int e = threadIdx.x + SNT * q, r = e >> 6, c = e & 63;
    if (r < rows && c < cols) {
      v[q] = (!diag || r <= c)
                 ? Elem<DT>::load((const typename Elem<DT>::T*)R + (r0 + r) * ldr + c0 + c)
                 : 0.0f;
      if (diag && ut && r == c) v[q] = 0.5f * (1.0f + v[q]);
    } else {
      v[q] = (diag && r == c) ? 1.0f : 0.0f;
    }
  }
#pragma unroll
  for (int q = 0; q < SB * SB / SNT; ++q) {
    const int e = threadIdx.x + SNT * q;
    S[(e >> 6) * SLD + (e & 63)] = v[q];
  }
  __syncthreads();
}

template <int DT>
__global__ __launch_bounds__(SNT) void trinv_diag128_kernel(const void* R, int64_t ldr, int64_t n,
                                                            float* Z, int64_t ldz, int safe,
                                                            int ut) {
  __shared__ float sA[SB * SLD];
  __shared__ float sZ1[SB * SLD];
  __shared__ float sZ2[SB * SLD];
  __shared__ float sX[SB * SLD];
  __shared__ float sT[TRINV_TMP];
  const int64_t k0 = (int64_t)blockIdx.x * (2 * SB);
  const int bt = (int)((n - k0) < 2 * SB ? (n - k0) : 2 * SB);
  const int b1 = bt < SB ? bt : SB, b2 = bt - b1;
  load_blk<DT>(sA, R, ldr, k0, k0, b1, b1, true, ut);
  sm_trinv64(sA, sZ1, sT, safe != 0);
  if (b2 > 0) {
    load_blk<DT>(sA, R, ldr, k0 + SB, k0 + SB, b2, b2, true, ut);
    sm_trinv64(sA, sZ2, sT, safe != 0);
    load_blk<DT>(sA, R, ldr, k0, k0 + SB, b1, b2, false, 0);   // R12 (b1 x b2)
    sm_gemm64<false, false>(sA, sZ2, sX, 1.0f, false);          // X = R12 Z22
    sm_gemm64<false, false>(sZ1, sX, sA, -1.0f, false);         // Z12 = -Z11 X
  }
  for (int e = threadIdx.x; e < SB * SB; e += SNT) {
    const int r = e >> 6, c = e & 63;
    if (r < b1 && c < b1) Z[(k0 + r) * ldz + k0 + c] = sZ1[r * SLD + c];
    if (r < b2 && c < b2) Z[(k0 + SB + r) * ldz + k0 + SB + c] = sZ2[r * SLD + c];
    if (r < b1 && c < b2) Z[(k0 + r) * ldz + k0 + SB + c] = sA[r * SLD + c];
  }
}

// ---------------------------------------------------------------------------
// Small fp32 GEMM, C_b = alpha * A_b B_b (row-major, batch b = blockIdx.y),
// one 64 x 64 output tile per workgroup: the products of a triangular
// inverse's first doubling levels, whose operands are too small to keep the
// 128-tile engine's few workgroups busy.  K runs in 64-wide chunks staged in
// LDS; the structural zeros of a triangular operand (tria / trib, TRI_UPPER
// or TRI_LOWER) are skipped by K range and masked in the chunks that cross
// its diagonal, so its stored other triangle is never read.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(SNT) void gemm64_kernel(int64_t M, int64_t N, int64_t K, float alpha,
                                                     const float* A, int64_t lda, int64_t bsa,
                                                     int tria, const float* B, int64_t ldb,
                                                     int64_t bsb, int trib, float* C, int64_t ldc,
                                                     int64_t bsc) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  __shared__ float sA[SB * SLD];
  __shared__ float sB[SB * SLD];
  const int64_t tiles_m = (M + SB - 1) / SB;
  const int64_t m0 = (int64_t)(blockIdx.x % tiles_m) * SB, n0 = (int64_t)(blockIdx.x / tiles_m) * SB;
  A += (int64_t)blockIdx.y * bsa;
  B += (int64_t)blockIdx.y * bsb;
  C += (int64_t)blockIdx.y * bsc;
  int64_t klo = 0, khi = K;
  if (tria == TRI_UPPER) klo = max(klo, m0);
  if (tria == TRI_LOWER) khi = min(khi, m0 + SB);
  if (trib == TRI_UPPER) khi = min(khi, n0 + SB);
  if (trib == TRI_LOWER) klo = max(klo, n0);
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int r = (wave >> 1) * 32 + l32;   // row of A this lane supplies
  const int c = (wave & 1) * 32 + l32;    // column of B this lane supplies
  f32x16 d;
#pragma unroll
  for (int i = 0; i < 16; ++i) d[i] = 0.0f;
  constexpr int PER = SB * SB / SNT;
  float va[PER], vb[PER];
  // chunk kc of A (rows m0.., columns kc..) and B (rows kc.., columns n0..)
  // into registers; the next chunk's loads fly while this one multiplies
  auto fetch = [&](int64_t kc) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = t + SNT * q, i = e >> 6, j = e & 63;
      const int64_t ar = m0 + i, ak = kc + j, bk = kc + i, bc = n0 + j;
      bool oka = ar < M && ak < khi && ak >= klo;
      if (tria == TRI_UPPER) oka = oka && ak >= ar;
      if (tria == TRI_LOWER) oka = oka && ak <= ar;
      bool okb = bc < N && bk < khi && bk >= klo;
      if (trib == TRI_UPPER) okb = okb && bk <= bc;
      if (trib == TRI_LOWER) okb = okb && bk >= bc;
      va[q] = oka ? A[ar * lda + ak] : 0.0f;
      vb[q] = okb ? B[bk * ldb + bc] : 0.0f;
    }
  };
  int64_t kc = (klo / SB) * SB;
  if (kc < khi) fetch(kc);
  for (; kc < khi; kc += SB) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = t + SNT * q;
      sA[(e >> 6) * SLD + (e & 63)] = va[q];
      sB[(e >> 6) * SLD + (e & 63)] = vb[q];
    }
    __syncthreads();
    if (kc + SB < khi) fetch(kc + SB);
#pragma unroll
    for (int st = 0; st < 32; ++st) {
      const int k = 32 * h + st;
      d = __builtin_amdgcn_mfma_f32_32x32x2f32(sA[r * SLD + k], sB[k * SLD + c], d, 0, 0, 0);
    }
    __syncthreads();
  }
  const int64_t col = n0 + (wave & 1) * 32 + l32;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = m0 + (wave >> 1) * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
    if (row < M && col < N) C[row * ldc + col] = alpha * d[i];
  }
}

// ---------------------------------------------------------------------------
// Small products with a fused epilogue (the 512 x 512 algebra of a CholeskyQR
// outer block), on fp32 MFMA:
//   v = alpha op(A) op(B) + beta1 C1 + beta2 C2 + gamma I
//   out = epi(v): SQ_PLAIN v, SQ_UP strict upper part + diag / 2, SQ_TRIU upper
//   part (strict lower zero in both)
// op(A) = A^T when ta (A stored K x M), op(B) = B^T when tb (B stored N x K);
// tria / trib describe op(A) / op(B) (their zero triangles are skipped by K
// range and masked).  alpha = 0 skips the product.  out2 (SQ_TRIU only,
// same ld as out) receives up(v) as well.  Up to SQ_BATCH independent
// products run in one launch (blockIdx.y selects the product).  outb receives an RNE
// bf16 copy, transposed (outb[j][i]) when outb_t.  With prev (same layout as
// out), any stored entry further than tol from prev's sets *flag = 1 (a
// convergence test).
//
// These products sit on the critical path of the fold while the far updates
// occupy most CUs, so the kernel is built for latency and a small footprint:
// a workgroup owns a 32 x 32 output tile (256 workgroups for 512 x 512),
// stages K in 32-wide chunks (12 KB of LDS, so eight workgroups fit a CU)
// with the next chunk's loads in flight during the current one, and its four
// waves split each chunk's K, reading k-contiguous fragments four at a time,
// before one cross-wave reduction.  The chunk width was measured on the
// 1024-column fold (pair of factor updates of the 4096 -> 11008, p = 16384
// step): 256: 26.5 ms, 128: 22.9, 64: 21.4, 32: 21.1 -- occupancy beats
// fewer dependent chunks.  With SQ_UP / SQ_TRIU, tiles wholly below the diagonal only
// store zeros and C1 / C2 are read on and above the diagonal only.
// ---------------------------------------------------------------------------
constexpr int SQ_T = 32;                 // output tile
constexpr int SQ_KC = 32;                // K chunk staged at a time
constexpr int SQ_LD = SQ_KC + 4;         // k-contiguous LDS rows; 4 mod 32 keeps
                                         // 8 rows' 16-byte reads on distinct banks
constexpr int SQ_PER = SQ_T * SQ_KC / 4 / SNT;   // float4 loads per thread and operand

// One K chunk of op(X) into registers: rows i0 + [0, 32) (row = tile row of
// op(A), or column n of op(B) staged as its transpose), k in [kbase, kbase +
// kext) (kext a multiple of 32, at most SQ_KC), zero outside [klo, khi), the
// matrix and its triangle.  kt: X is stored with k along rows (op(X)[i][k] =
// X[k * ld + i]); otherwise op(X)[i][k] = X[i * ld + k].  keep_ge / keep_le
// keep k >= i / k <= i.  vec: 16-byte loads are aligned.  Each thread loads
// SQ_PER groups of 4 consecutive elements along the stored contiguous index.
__device__ __forceinline__ void sq_load(float4 (&v)[SQ_PER], const float* X, int64_t ld, bool kt,
                                        int64_t i0, int64_t ilim, int64_t kbase, int kext,
                                        int64_t klo, int64_t khi, int keep_ge, int keep_le,
                                        bool vec) {
  const int t = threadIdx.x;
#pragma unroll
  for (int q = 0; q < SQ_PER; ++q) {
    const int e = t + SNT * q;
    int ii, kk;   // tile-relative row, k of the group's first element
    if (!kt) { ii = e / (SQ_KC / 4); kk = (e % (SQ_KC / 4)) * 4; }
    else { kk = e / (SQ_T / 4); ii = (e % (SQ_T / 4)) * 4; }
    float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (kk < kext) {
      const int64_t gi = i0 + ii, gk = kbase + kk;
      if (!kt) {
        if (gi < ilim) {
          const float* g = X + gi * ld + gk;
          if (vec && gk + 3 < khi && gk >= klo) {
            const float4 w = *(const float4*)g;
            x[0] = w.x, x[1] = w.y, x[2] = w.z, x[3] = w.w;
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u)
              if (gk + u >= klo && gk + u < khi) x[u] = g[u];
          }
        }
      } else {
        if (gk >= klo && gk < khi) {
          const float* g = X + gk * ld + gi;
          if (vec && gi + 3 < ilim) {
            const float4 w = *(const float4*)g;
            x[0] = w.x, x[1] = w.y, x[2] = w.z, x[3] = w.w;
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u)
              if (gi + u < ilim) x[u] = g[u];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t ri = i0 + ii + (kt ? u : 0), rk = kbase + kk + (kt ? 0 : u);
        if ((keep_ge && rk < ri) || (keep_le && rk > ri)) x[u] = 0.0f;
      }
    }
    v[q] = make_float4(x[0], x[1], x[2], x[3]);
  }
}

// The registers of sq_load into the k-contiguous LDS tile S[row][k - kbase]
__device__ __forceinline__ void sq_store(float* S, const float4 (&v)[SQ_PER], bool kt, int kext) {
  const int t = threadIdx.x;
#pragma unroll
  for (int q = 0; q < SQ_PER; ++q) {
    const int e = t + SNT * q;
    if (!kt) {
      const int ii = e / (SQ_KC / 4), kk = (e % (SQ_KC / 4)) * 4;
      if (kk < kext) *(float4*)&S[ii * SQ_LD + kk] = v[q];
    } else {
      const int kk = e / (SQ_T / 4), ii = (e % (SQ_T / 4)) * 4;
      if (kk < kext) {
        S[(ii + 0) * SQ_LD + kk] = v[q].x;
        S[(ii + 1) * SQ_LD + kk] = v[q].y;
        S[(ii + 2) * SQ_LD + kk] = v[q].z;
        S[(ii + 3) * SQ_LD + kk] = v[q].w;
      }
    }
  }
}

__global__ __launch_bounds__(SNT) void sqmm_kernel(SqmmBatch batch) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  const SqmmArgs& a = batch.a[blockIdx.y];
  if ((int64_t)blockIdx.x >= ((a.M + SQ_T - 1) / SQ_T) * ((a.N + SQ_T - 1) / SQ_T)) return;
  // the two staged operands, and after the K loop the cross-wave partial
  // sums of waves 1..3 (3 x 16 x 64 floats)
  constexpr int SQ_SMEM = 2 * SQ_T * SQ_LD > 3 * 16 * 64 ? 2 * SQ_T * SQ_LD : 3 * 16 * 64;
  __shared__ __attribute__((aligned(16))) float smem[SQ_SMEM];
  float* const sA = smem;
  float* const sB = smem + SQ_T * SQ_LD;
  const int64_t tiles_m = (a.M + SQ_T - 1) / SQ_T;
  const int64_t m0 = (int64_t)(blockIdx.x % tiles_m) * SQ_T,
                n0 = (int64_t)(blockIdx.x / tiles_m) * SQ_T;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t col = n0 + l32;
  if (a.epi != SQ_PLAIN && m0 > n0 + SQ_T - 1) {   // strictly below the diagonal
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t row = m0 + (i >> 2) * 8 + h * 4 + (i & 3);
        if (row < a.M && col < a.N) {
          a.out[row * a.ldo + col] = 0.0f;
          if (a.out2) a.out2[row * a.ldo + col] = 0.0f;
          if (a.outb) a.outb[a.outb_t ? col * a.ldob + row : row * a.ldob + col] = 0;
        }
      }
    }
    return;
  }
  int64_t klo = 0, khi = a.alpha != 0.0f ? a.K : 0;
  if (a.tria == TRI_UPPER) klo = max(klo, m0);
  if (a.tria == TRI_LOWER) khi = min(khi, m0 + SQ_T);
  if (a.trib == TRI_UPPER) khi = min(khi, n0 + SQ_T);
  if (a.trib == TRI_LOWER) klo = max(klo, n0);
  f32x16 d;
#pragma unroll
  for (int i = 0; i < 16; ++i) d[i] = 0.0f;
  if (klo < khi) {
    // K in chunks of SQ_KC; the next chunk's loads fly while this one
    // multiplies.  Wave w takes k in [w kq, (w + 1) kq) of the chunk, lane
    // half h the halves of that range, four steps per 16-byte read.
    const int64_t k0 = klo & ~(int64_t)3;
    float4 va[SQ_PER], vb[SQ_PER];
    auto kext_of = [&](int64_t kb) {
      const int kr = (int)min((int64_t)SQ_KC, khi - kb);
      return ((kr + 31) / 32) * 32;
    };
    int kext = kext_of(k0);
    sq_load(va, a.A, a.lda, a.ta != 0, m0, a.M, k0, kext, klo, khi, a.tria == TRI_UPPER,
            a.tria == TRI_LOWER, a.vec_a != 0);
    // op(B) staged as its transpose: row = column n of op(B)
    sq_load(vb, a.B, a.ldb, a.tb == 0, n0, a.N, k0, kext, klo, khi, a.trib == TRI_LOWER,
            a.trib == TRI_UPPER, a.vec_b != 0);
    for (int64_t kb = k0; kb < khi; kb += SQ_KC) {
      if (kb != k0) __syncthreads();   // every wave is done with the last chunk
      sq_store(sA, va, a.ta != 0, kext);
      sq_store(sB, vb, a.tb == 0, kext);
      __syncthreads();
      const int kq = kext / 4, half = kq / 2;
      if (kb + SQ_KC < khi) {
        kext = kext_of(kb + SQ_KC);
        sq_load(va, a.A, a.lda, a.ta != 0, m0, a.M, kb + SQ_KC, kext, klo, khi,
                a.tria == TRI_UPPER, a.tria == TRI_LOWER, a.vec_a != 0);
        sq_load(vb, a.B, a.ldb, a.tb == 0, n0, a.N, kb + SQ_KC, kext, klo, khi,
                a.trib == TRI_LOWER, a.trib == TRI_UPPER, a.vec_b != 0);
      }
      const int kw = wave * kq + h * half;
      for (int st = 0; st < half; st += 4) {
        const float4 av = *(const float4*)&sA[l32 * SQ_LD + kw + st];
        const float4 bv = *(const float4*)&sB[l32 * SQ_LD + kw + st];
        d = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, d, 0, 0, 0);
      }
    }
    // cross-wave sum into wave 0 (smem is free once every wave is past its reads)
    __syncthreads();
    if (wave > 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) smem[((wave - 1) * 16 + i) * 64 + lane] = d[i];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        d[i] += smem[i * 64 + lane] + smem[(16 + i) * 64 + lane] + smem[(32 + i) * 64 + lane];
    }
  }
  if (wave != 0) return;
  float dm = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = m0 + (i >> 2) * 8 + h * 4 + (i & 3);
    if (row >= a.M || col >= a.N) continue;
    const bool keep = a.epi == SQ_PLAIN || row <= col;
    float v = 0.0f;
    if (keep) {
      v = a.alpha * d[i];
      if (a.C1) v += a.beta1 * a.C1[row * a.ld1 + col];
      if (a.C2) v += a.beta2 * a.C2[row * a.ld2 + col];
      if (row == col) v += a.gamma;
      if (a.epi == SQ_UP && row == col) v *= 0.5f;
    }
    a.out[row * a.ldo + col] = v;
    if (a.out2) a.out2[row * a.ldo + col] = (row < col) ? v : (row == col ? 0.5f * v : 0.0f);
    if (a.outb) a.outb[a.outb_t ? col * a.ldob + row : row * a.ldob + col] = f32_to_bf16(v);
    if (a.prev) dm = fmaxf(dm, fabsf(v - a.prev[row * a.ldo + col]));
  }
  if (a.prev) {
    for (int o = 32; o > 0; o >>= 1) dm = fmaxf(dm, __shfl_xor(dm, o));
    if (lane == 0 && !(dm <= a.tol)) *a.flag = 1;
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
int launch_sqmm(hipStream_t s, const SqmmArgs* args, int count) {
  if (count < 1 || count > SQ_BATCH) {
    set_error("sqmm: batch size out of range");
    return IFK_ERR_INVALID;
  }
  SqmmBatch b;
  int64_t tiles = 0;
  for (int i = 0; i < count; ++i) {
    const SqmmArgs& a0 = args[i];
    if (a0.M < 0 || a0.N < 0 || a0.K < 0 || !a0.out || (a0.prev && !a0.flag) ||
        (a0.out2 && a0.epi != SQ_TRIU)) {
      set_error("sqmm: invalid arguments");
      return IFK_ERR_INVALID;
    }
    b.a[i] = a0;
    // 16-byte operand loads need 16-byte aligned rows
    b.a[i].vec_a = a0.A && ((uintptr_t)a0.A & 15) == 0 && a0.lda % 4 == 0;
    b.a[i].vec_b = a0.B && ((uintptr_t)a0.B & 15) == 0 && a0.ldb % 4 == 0;
    tiles = std::max<int64_t>(tiles, cdiv(a0.M, (int64_t)SQ_T) * cdiv(a0.N, (int64_t)SQ_T));
  }
  if (tiles == 0) return IFK_OK;
  if (tiles > 0x7fffffffLL) {
    set_error("sqmm: grid too large");
    return IFK_ERR_INVALID;
  }
  hipLaunchKernelGGL(sqmm_kernel, dim3((unsigned)tiles, (unsigned)count), dim3(SNT), 0, s, b);
  return check_launch("sqmm");
}

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

int launch_cholb(hipStream_t s, float* A, int64_t lda, int n, float* U, int64_t ldu, float* Zd,
                 float* dref, float tol, int* flag, float* M, int64_t ldm, bool dref_in,
                 int batch, CholbStrides bs) {
  if (n < 1 || n > CHOLB_MAX || lda < n || ldu < n || (M && ldm < n) || batch < 1 ||
      batch > 65535) {
    set_error("cholb: size out of range");
    return IFK_ERR_INVALID;
  }
  const int nb = (n + SB - 1) / SB;
  // launch profiler: the algorithmic work of the factor (n^3 / 3) and, with M,
  // its inverse (n^3 / 3 more) spread evenly over the launches, the bytes of
  // A's upper triangle read and of U (and M) written
  const int launches = M ? nb + 1 : nb;
  const double nn = (double)n;
  const double fl = (M ? 2.0 : 1.0) * nn * nn * nn / 3.0 * batch / launches;
  const double by = (M ? 3.0 : 2.0) * nn * nn / 2.0 * 4.0 * batch / launches;
  void* pr = prof_kernel_begin(s, KVID_CHOLB_FIRST, fl, by, n, n, 0);
  hipLaunchKernelGGL(cholb_first_kernel, dim3(1, (unsigned)batch), dim3(SNT), 0, s, A, lda, n, U,
                     ldu, Zd, dref, tol, flag, M, ldm, dref_in ? 1 : 0, bs);
  prof_kernel_end(pr, s);
  if (int rc = check_launch("cholb_first")) return rc;
  // step k: the (i, j) pairs k < i <= j (m (m + 1) / 2 of them, m = nb - 1 - k),
  // then with M the k + 1 blocks of M's column block k and the k m partial
  // sums of its later column blocks (column block 0 comes from cholb_first;
  // the last takes one more launch, k = nb - 1, of M blocks only)
  for (int k = 0; k < nb; ++k) {
    const int m = nb - 1 - k;
    const int wgs = m * (m + 1) / 2 + ((M && k > 0) ? k + 1 + k * m : 0);
    if (wgs == 0) continue;
    void* ps = prof_kernel_begin(s, KVID_CHOLB_STEP, fl, by, n, n, k);
    hipLaunchKernelGGL(cholb_step_kernel, dim3((unsigned)wgs, (unsigned)batch), dim3(SNT), 0, s, A,
                       lda, n, U, ldu, Zd, dref, tol, flag, k, M, ldm, bs);
    prof_kernel_end(ps, s);
    if (int rc = check_launch("cholb_step")) return rc;
  }
  return IFK_OK;
}

static unsigned ew_grid(int64_t total) {
  int64_t g = cdiv(total, 256);
  if (g < 1) g = 1;
  if (g > 1024) g = 1024;
  return (unsigned)g;
}

int launch_split_bf16(hipStream_t s, const float* src, int64_t lds, int64_t rows, int64_t cols,
                      bf16_t* hi, bf16_t* lo, int64_t ldo, bool trans) {
  if (rows <= 0 || cols <= 0) return IFK_OK;
  hipLaunchKernelGGL(split_bf16_kernel, dim3(ew_grid(rows * cols)), dim3(256), 0, s, src, lds, rows,
                     cols, hi, lo, ldo, trans ? 1 : 0);
  return check_launch("split_bf16");
}

int launch_status_merge(hipStream_t s, int* status, const int* flag) {
  hipLaunchKernelGGL(status_merge_kernel, dim3(1), dim3(64), 0, s, status, flag);
  return check_launch("status_merge");
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
                      float* Z, int64_t ldz, int safe, bf16_t* Zb, bf16_t* ZTb, int64_t ldb) {
  if (int rc = check_b(nb, "trinv_diag")) return rc;
  const unsigned nblk = (unsigned)cdiv(n, nb);
  if (rdt == DT_F32)
    hipLaunchKernelGGL(trinv_diag_kernel<DT_F32>, dim3(nblk), dim3(SNT), 0, s, R, ldr, n, nb, Z,
                       ldz, safe, Zb, ZTb, ldb);
  else
    hipLaunchKernelGGL(trinv_diag_kernel<DT_BF16>, dim3(nblk), dim3(SNT), 0, s, R, ldr, n, nb, Z,
                       ldz, safe, Zb, ZTb, ldb);
  return check_launch("trinv_diag");
}

int launch_trinv_diag128(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* Z,
                         int64_t ldz, int safe, int ut) {
  if (n <= 0) return IFK_OK;
  const unsigned nblk = (unsigned)cdiv(n, (int64_t)(2 * SB));
  if (rdt == DT_F32)
    hipLaunchKernelGGL(trinv_diag128_kernel<DT_F32>, dim3(nblk), dim3(SNT), 0, s, R, ldr, n, Z, ldz,
                       safe, ut);
  else
    hipLaunchKernelGGL(trinv_diag128_kernel<DT_BF16>, dim3(nblk), dim3(SNT), 0, s, R, ldr, n, Z, ldz,
                       safe, ut);
  return check_launch("trinv_diag128");
}

int launch_gemm64(hipStream_t s, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
                  int64_t lda, int64_t bsa, int tria, const float* B, int64_t ldb, int64_t bsb,
                  int trib, float* C, int64_t ldc, int64_t bsc, int batch) {
  if (M <= 0 || N <= 0) return IFK_OK;
  const int64_t tiles = cdiv(M, (int64_t)SB) * cdiv(N, (int64_t)SB);
  if (tiles > 0x7fffffffLL || batch < 1 || batch > 65535) {
    set_error("gemm64: grid too large");
    return IFK_ERR_INVALID;
  }
  hipLaunchKernelGGL(gemm64_kernel, dim3((unsigned)tiles, (unsigned)batch), dim3(SNT), 0, s, M, N,
                     K, alpha, A, lda, bsa, tria, B, ldb, bsb, trib, C, ldc, bsc);
  return check_launch("gemm64");
}

}  // namespace ifk
