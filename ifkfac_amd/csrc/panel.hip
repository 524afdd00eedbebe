// Streaming kernels of one panel step of the fold (see linalg.hip).  They run
// over the p_e rows of the working matrix C in parallel and leave the
// b x b / b x nr reductions to the single-workgroup kernels of small.hip:
//
//   gram_partial   part[s][cb] = A_s^T B_s,cb  (64 x 64 per 128-row slab s
//                  and 64-column block cb of B) -- G1 = X_p^T X_p, then
//                  G2 = Q2^T Q2 and Q2^T C_rest
//   gram_reduce    G[cb] = sum_s part[s][cb], in slab order (deterministic)
//   apply_m        Q2 = X_p M1 (skipped for a flagged panel: the Householder
//                  fallback has written its reflectors into Q2)
//   panel_update   Y = Q2 N into the outer block's reflector store and
//                  C_rest -= Q2 NW (NW = N W from panel_wcomp)
//
// All products run on fp32 MFMA (v_mfma_f32_32x32x2f32, fp32 accumulation):
// the panel sits on the critical path of the factorisation and its
// reflectors must be orthogonal to fp32 working precision.  Row slabs and
// tiles are staged through LDS with padded strides; the 64 x 64 output tile
// of a workgroup is split in four 32 x 32 quadrants, one per wave.
#include "common.h"
#include "kernels.h"

namespace ifk {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int PT = 64;        // panel / tile width
constexpr int PNT = 256;      // threads per workgroup (4 waves)
constexpr int GSLAB = 128;    // rows per slab of the Gram kernel (one LDS sweep)
constexpr int TLD = PT + 4;   // LDS row stride (floats)

// Load rows [r0, r0 + nr) x columns [0, 64) of a row-major matrix into an LDS
// tile with row stride TLD; columns >= w and rows >= rmax read as zero.
__device__ __forceinline__ void load_tile(float* S, const float* g, int64_t ld, int64_t r0,
                                          int nr, int64_t rmax, int w) {
  for (int e = threadIdx.x; e < nr * PT; e += PNT) {
    const int r = e >> 6, c = e & 63;
    const int64_t gr = r0 + r;
    S[r * TLD + c] = (gr < rmax && c < w) ? g[gr * ld + c] : 0.0f;
  }
}

// acc += S1^T S2 over `rows` rows of two LDS tiles (k = row); wave quadrant
// (w >> 1, w & 1), lane (l32, h) supplies rows k = 2 s + h.
__device__ __forceinline__ void mfma_tn(const float* S1, const float* S2, int rows, f32x16& d) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int i = (wave >> 1) * 32 + l32, j = (wave & 1) * 32 + l32;
#pragma unroll 8
  for (int s = 0; s < rows / 2; ++s) {
    const int k = 2 * s + h;
    d = __builtin_amdgcn_mfma_f32_32x32x2f32(S1[k * TLD + i], S2[k * TLD + j], d, 0, 0, 0);
  }
}

// d = S1 M over 64 x 64 LDS tiles (S1 rows x k, M k x cols); lane (l32, h)
// supplies k = 32 h + s.
__device__ __forceinline__ void mfma_nn(const float* S1, const float* M, f32x16& d) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int i = (wave >> 1) * 32 + l32, j = (wave & 1) * 32 + l32;
#pragma unroll 8
  for (int s = 0; s < 32; ++s) {
    const int k = 32 * h + s;
    d = __builtin_amdgcn_mfma_f32_32x32x2f32(S1[i * TLD + k], M[k * TLD + j], d, 0, 0, 0);
  }
}

__device__ __forceinline__ void zero16(f32x16& d) {
#pragma unroll
  for (int r = 0; r < 16; ++r) d[r] = 0.0f;
}

// Row / column of accumulator element r of this lane in the 64 x 64 tile.
__device__ __forceinline__ int acc_row(int r) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  return (wave >> 1) * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
}
__device__ __forceinline__ int acc_col() {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  return (wave & 1) * 32 + (lane & 31);
}

}  // namespace

// part[(s * ncb + cb) * 4096 + i * 64 + j] = sum over the rows r of slab s
// (GSLAB rows, loaded into LDS in one sweep) of A[r][i] * Bcb[r][j], with
// Bcb = B0 (cb == 0, when B0 is given) or the 64-column block
// (cb - (B0 ? 1 : 0)) of B1.  Columns beyond ka / w0 / w1 are zero.
__global__ __launch_bounds__(PNT) void gram_partial_kernel(const float* A, int64_t lda, int ka,
                                                           const float* B0, int64_t ldb0, int w0,
                                                           const float* B1, int64_t ldb1, int w1,
                                                           int64_t pe, float* part, int ncb) {
  __shared__ float sA[GSLAB * TLD];
  __shared__ float sB[GSLAB * TLD];
  const int s = blockIdx.x, cb = blockIdx.y;
  const float* B;
  int64_t ldb;
  int wb;
  if (B0 != nullptr && cb == 0) {
    B = B0;
    ldb = ldb0;
    wb = w0;
  } else {
    const int blk = cb - (B0 != nullptr ? 1 : 0);
    B = B1 + (int64_t)blk * PT;
    ldb = ldb1;
    wb = w1 - blk * PT;
  }
  const int64_t r0 = (int64_t)s * GSLAB;
  load_tile(sA, A, lda, r0, GSLAB, pe, ka);
  load_tile(sB, B, ldb, r0, GSLAB, pe, wb);
  __syncthreads();
  f32x16 d;
  zero16(d);
  mfma_tn(sA, sB, GSLAB, d);
  float* out = part + ((size_t)s * ncb + cb) * (PT * PT);
  const int j = acc_col();
#pragma unroll
  for (int r = 0; r < 16; ++r) out[acc_row(r) * PT + j] = d[r];
}

// G[cb * 4096 + e] = sum over s < nslab of part[(s * ncb + cb) * 4096 + e],
// in slab order (deterministic).
__global__ __launch_bounds__(PNT) void gram_reduce_kernel(const float* part, int nslab, int ncb,
                                                          float* G) {
  const int64_t idx = (int64_t)blockIdx.x * PNT + threadIdx.x;   // over ncb * 4096
  if (idx >= (int64_t)ncb * PT * PT) return;
  const int64_t cb = idx / (PT * PT), e = idx % (PT * PT);
  const float* p0 = part + cb * (PT * PT) + e;
  const int64_t stride = (int64_t)ncb * PT * PT;
  float acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = 0.0f;
  int sl = 0;
  for (; sl + 8 <= nslab; sl += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] += p0[(int64_t)(sl + u) * stride];
  }
  for (int u = 0; sl < nslab; ++sl, ++u) acc[u] += p0[(int64_t)sl * stride];
  G[idx] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

// Q2[r][:] = X[r][0:b] M (M b x b in ld b), r < pe, Q2 of ld 64 (columns >= b
// written as zero).  Nothing is done when *flag is set.
__global__ __launch_bounds__(PNT) void apply_m_kernel(const float* X, int64_t ldx, int64_t pe,
                                                      int b, const float* M, float* Q2,
                                                      const int* flag) {
  if (*flag) return;
  __shared__ float sX[PT * TLD];
  __shared__ float sM[PT * TLD];
  const int64_t r0 = (int64_t)blockIdx.x * PT;
  load_tile(sX, X, ldx, r0, PT, pe, b);
  load_tile(sM, M, b, 0, PT, b, b);
  __syncthreads();
  f32x16 d;
  zero16(d);
  mfma_nn(sX, sM, d);
  const int j = acc_col();
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t gr = r0 + acc_row(r);
    if (gr < pe) Q2[gr * PT + j] = d[r];
  }
}

// Panel update for the 64-row tile rb (the Q2 tile is loaded once):
//   Y[r][0:b] = Q2[r][:] N                              (Y of ld ldy; RNE bf16
//                                                        copy into Yb if given)
//   C[r][c] -= Q2[r][:] NW[:, c] for the nr columns of C_rest (NW of ld ldnw)
__global__ __launch_bounds__(PNT) void panel_update_kernel(const float* Q2, int64_t pe, int b,
                                                           const float* N, float* Y, int64_t ldy,
                                                           bf16_t* Yb, const float* NW,
                                                           int64_t ldnw, float* C, int64_t ldc,
                                                           int nr) {
  __shared__ float sQ[PT * TLD];
  __shared__ float sM[PT * TLD];
  const int64_t r0 = (int64_t)blockIdx.x * PT;
  const int j = acc_col();
  load_tile(sQ, Q2, PT, r0, PT, pe, PT);
  const int nblk = (nr + PT - 1) / PT;
  for (int cb = 0; cb <= nblk; ++cb) {
    int w;
    if (cb == 0) {
      load_tile(sM, N, b, 0, PT, b, b);
      w = b;
    } else {
      w = nr - (cb - 1) * PT;
      if (w > PT) w = PT;
      load_tile(sM, NW + (cb - 1) * PT, ldnw, 0, PT, PT, w);
    }
    __syncthreads();
    f32x16 d;
    zero16(d);
    mfma_nn(sQ, sM, d);
    if (j < w) {
      if (cb == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t gr = r0 + acc_row(r);
          if (gr < pe) {
            Y[gr * ldy + j] = d[r];
            if (Yb) Yb[gr * ldy + j] = f32_to_bf16(d[r]);
          }
        }
      } else {
        float* Cb = C + (cb - 1) * PT;
        float cur[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t gr = r0 + acc_row(r);
          cur[r] = (gr < pe) ? Cb[gr * ldc + j] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t gr = r0 + acc_row(r);
          if (gr < pe) Cb[gr * ldc + j] = cur[r] - d[r];
        }
      }
    }
    __syncthreads();   // sM is reloaded for the next block
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
int gram_slabs(int64_t pe) { return (int)cdiv(pe > 0 ? pe : 1, (int64_t)GSLAB); }

int launch_gram(hipStream_t s, const float* A, int64_t lda, int ka, const float* B0, int64_t ldb0,
                int w0, const float* B1, int64_t ldb1, int w1, int64_t pe, float* part, float* G,
                int* ncb_out) {
  if (ka > PT || (B0 && w0 > PT)) {
    set_error("gram: block wider than 64");
    return IFK_ERR_INVALID;
  }
  const int ns = gram_slabs(pe);
  const int ncb = (B0 ? 1 : 0) + (int)cdiv((int64_t)(w1 > 0 ? w1 : 0), (int64_t)PT);
  if (ncb > PANEL_MAX_CB) {
    set_error("gram: too many column blocks");
    return IFK_ERR_INVALID;
  }
  *ncb_out = ncb;
  if (ncb == 0) return IFK_OK;
  hipLaunchKernelGGL(gram_partial_kernel, dim3(ns, ncb), dim3(PNT), 0, s, A, lda, ka, B0, ldb0,
                     w0, B1, ldb1, w1, pe, part, ncb);
  if (int rc = check_launch("gram_partial")) return rc;
  const int64_t total = (int64_t)ncb * PT * PT;
  hipLaunchKernelGGL(gram_reduce_kernel, dim3((unsigned)cdiv(total, (int64_t)PNT)), dim3(PNT), 0, s,
                     part, ns, ncb, G);
  return check_launch("gram_reduce");
}

int launch_apply_m(hipStream_t s, const float* X, int64_t ldx, int64_t pe, int b, const float* M,
                   float* Q2, const int* flag) {
  if (pe <= 0) return IFK_OK;
  hipLaunchKernelGGL(apply_m_kernel, dim3((unsigned)cdiv(pe, (int64_t)PT)), dim3(PNT), 0, s, X,
                     ldx, pe, b, M, Q2, flag);
  return check_launch("apply_m");
}

int launch_panel_update(hipStream_t s, const float* Q2, int64_t pe, int b, const float* N,
                        float* Y, int64_t ldy, bf16_t* Yb, const float* NW, int64_t ldnw, float* C,
                        int64_t ldc, int nr) {
  if (pe <= 0) return IFK_OK;
  hipLaunchKernelGGL(panel_update_kernel, dim3((unsigned)cdiv(pe, (int64_t)PT)), dim3(PNT), 0, s,
                     Q2, pe, b, N, Y, ldy, Yb, NW, ldnw, C, ldc, nr);
  return check_launch("panel_update");
}

}  // namespace ifk
