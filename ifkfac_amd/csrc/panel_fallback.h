// Robust TPQRT panel by Householder reflections (LAPACK dlarfg convention),
// the fallback of the CholeskyQR2 panel for rank-deficient or ill-conditioned
// panels.  The reflectors' X parts go to Y (p_e x 64, ld 64, columns >= b
// zero) and R's diagonal block P_top (at ldr) is replaced by R_new.  The panel
// X_p is read from the transposed working matrix (XpT: b x p_e, ld ldx).  One
// workgroup of 256 threads walks the b columns; norms and dot products over
// the p_e rows are wave-shuffle reductions.  sP: LDS of 64 * 65 floats, aux:
// LDS of at least 5 * 64 + 3 floats.
#pragma once
#include "common.h"

namespace ifk {

__device__ __forceinline__ void panel_hh_fallback(float* Ptop, int64_t ldr, const float* XpT,
                                                  int64_t ldx, int64_t pe, int b, float* Y,
                                                  float* sP, float* aux) {
  constexpr int B = 64, LD = B + 1, NT = 256;
  constexpr int64_t ldy = B;
  float* red = aux;            // [4][64]
  float* wv = aux + 4 * B;     // [64]
  float* scal = aux + 5 * B;   // [3]
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  for (int e = t; e < B * B; e += NT) {
    const int r = e >> 6, c = e & 63;
    sP[r * LD + c] = (r < b && c < b && r <= c) ? Ptop[(int64_t)r * ldr + c] : 0.0f;
  }
  for (int64_t e = t; e < pe * B; e += NT) {
    const int64_t r = e / B;
    const int c = (int)(e % B);
    Y[r * ldy + c] = (c < b) ? XpT[(int64_t)c * ldx + r] : 0.0f;
  }
  __syncthreads();
  for (int j = 0; j < b; ++j) {
    float part = 0.0f;
    for (int64_t r = t; r < pe; r += NT) {
      const float v = Y[r * ldy + j];
      part += v * v;
    }
    for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o);
    if (lane == 0) red[wave * B] = part;
    __syncthreads();
    if (t == 0) {
      const float xn2 = red[0] + red[B] + red[2 * B] + red[3 * B];
      const float alpha = sP[j * LD + j];
      if (!(xn2 > 0.0f)) {
        // Nothing below the diagonal: reflect row j alone (v = e_j, tau = 2),
        // which is what the UT transform of a zero y_j encodes (T_jj = 2).
        scal[0] = 2.0f;
        scal[1] = 0.0f;
        scal[2] = -alpha;
      } else {
        const float nrm = sqrtf(alpha * alpha + xn2);
        const float beta = (alpha >= 0.0f) ? -nrm : nrm;
        scal[0] = (beta - alpha) / beta;
        scal[1] = 1.0f / (alpha - beta);
        scal[2] = beta;
      }
    }
    __syncthreads();
    const float tau = scal[0], sc = scal[1];
    for (int64_t r = t; r < pe; r += NT) Y[r * ldy + j] *= sc;
    __syncthreads();
    float acc[B];
#pragma unroll
    for (int c = 0; c < B; ++c) acc[c] = 0.0f;
    for (int64_t r = t; r < pe; r += NT) {
      const float y = Y[r * ldy + j];
#pragma unroll
      for (int c = 0; c < B; ++c)
        if (c > j && c < b) acc[c] += y * Y[r * ldy + c];
    }
#pragma unroll
    for (int c = 0; c < B; ++c) {
      if (c > j && c < b) {
        float v = acc[c];
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
        if (lane == 0) red[wave * B + c] = v;
      }
    }
    __syncthreads();
    for (int c = j + 1 + t; c < b; c += NT)
      wv[c] = sP[j * LD + c] + red[c] + red[B + c] + red[2 * B + c] + red[3 * B + c];
    __syncthreads();
    for (int c = j + 1 + t; c < b; c += NT) sP[j * LD + c] -= tau * wv[c];
    for (int64_t e = t; e < pe * (b - j - 1); e += NT) {
      const int64_t r = e / (b - j - 1);
      const int c = j + 1 + (int)(e % (b - j - 1));
      Y[r * ldy + c] -= tau * wv[c] * Y[r * ldy + j];
    }
    if (t == 0) sP[j * LD + j] = scal[2];
    __syncthreads();
  }
  for (int e = t; e < b * b; e += NT) {
    const int i = e / b, c = e - i * b;
    Ptop[(int64_t)i * ldr + c] = (i <= c) ? sP[i * LD + c] : 0.0f;
  }
}

}  // namespace ifk
