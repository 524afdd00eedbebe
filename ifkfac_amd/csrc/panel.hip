// Streaming kernels of one panel step of the fold (see linalg.hip).  They run
// over the p_e rows of the working matrix in parallel and leave the b x b /
// b x nr reductions to the single-workgroup kernels of small.hip.
//
// The fold keeps its working matrix transposed: CT = C^T (n x p, row stride
// ldc), so a panel X_p = C[:, c0:c1] is the contiguous row block CT[c0:c1, :]
// and every large product of the outer update reads K-contiguous operands.
// Q2 (p x 64) and the reflector store Y (p x 512) stay row-major.
//
//   gram_partial   part[s][cb] = A_s^T B_s,cb  (64 x 64 per 128-row slab s
//                  and 64-column block cb of B) -- G1 = X_p^T X_p, then
//                  G2 = Q2^T Q2 and Q2^T C_rest
//   gram_reduce    G[cb] = sum_s part[s][cb], in slab order (deterministic)
//   apply_m        Q2 = X_p M1, or for a flagged panel the Householder
//                  fallback (reflectors into Q2, R_new into P_top)
//   panel_update   Y = Q2 N into the outer block's reflector store and
//                  CT_rest -= (Q2 NW)^T (NW = N W from panel_hrw)
//
// All products run on fp32 MFMA (v_mfma_f32_32x32x2f32, fp32 accumulation):
// the panel sits on the critical path of the factorisation and its
// reflectors must be orthogonal to fp32 working precision.  Operand tiles
// are staged through LDS "column-major" (S[c * ldS + r], odd ldS): reads of
// the transposed working matrix are coalesced along r, writes of row-major
// tiles hit distinct banks, and MFMA fragments read consecutive r.  The
// 64 x 64 output tile of a workgroup is split in four 32 x 32 quadrants, one
// per wave.
#include "common.h"
#include "kernels.h"
#include "panel_fallback.h"

namespace ifk {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int PT = 64;        // panel / tile width
constexpr int PNT = 256;      // threads per workgroup (4 waves)
constexpr int GSLAB = 128;    // rows per slab of the Gram kernel (one LDS sweep)
constexpr int LG = GSLAB + 1; // column stride of a slab tile in LDS (floats)
constexpr int LT = PT + 1;    // column stride of a 64-row tile in LDS
constexpr int TLD = PT + 4;   // row stride of a row-major 64 x 64 LDS tile

// Rows [r0, r0 + NR) of a p x 64 operand view into LDS as S[c * ldS + r];
// columns >= w and rows >= rmax read as zero.  TS: the operand is stored
// transposed (element (r, c) at g[c * ld + r], the working matrix); else
// row-major (g[r * ld + c]).  All loads of a thread are issued before the
// first LDS write (one memory latency per tile, not one per element).
template <bool TS, int NR>
__device__ __forceinline__ void load_cm(float* S, int ldS, const float* g, int64_t ld, int64_t r0,
                                        int64_t rmax, int w) {
  constexpr int PER = NR * PT / PNT;
  float v[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = threadIdx.x + PNT * q;
    int r, c;
    if constexpr (TS) {
      c = e / NR;
      r = e - c * NR;
    } else {
      r = e >> 6;
      c = e & 63;
    }
    const int64_t gr = r0 + r;
    v[q] = (gr < rmax && c < w) ? (TS ? g[(int64_t)c * ld + gr] : g[gr * ld + c]) : 0.0f;
  }
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = threadIdx.x + PNT * q;
    int r, c;
    if constexpr (TS) {
      c = e / NR;
      r = e - c * NR;
    } else {
      r = e >> 6;
      c = e & 63;
    }
    S[c * ldS + r] = v[q];
  }
}

// Row-major 64 x 64 tile (M b x b in ld, or a 64-column block) into LDS with
// row stride TLD; rows >= rows_ok and columns >= w read as zero.
__device__ __forceinline__ void load_rm(float* S, const float* g, int64_t ld, int rows_ok, int w) {
  constexpr int PER = PT * PT / PNT;
  float v[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = threadIdx.x + PNT * q, r = e >> 6, c = e & 63;
    v[q] = (r < rows_ok && c < w) ? g[(int64_t)r * ld + c] : 0.0f;
  }
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = threadIdx.x + PNT * q;
    S[(e >> 6) * TLD + (e & 63)] = v[q];
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
// Bcb = B0 (cb == 0, when B0 is given; row-major) or the 64-column block
// (cb - (B0 ? 1 : 0)) of B1 (stored transposed).  A is stored transposed when
// A_TS.  Columns beyond ka / w0 / w1 are zero.
template <bool A_TS>
__global__ __launch_bounds__(PNT) void gram_partial_kernel(const float* A, int64_t lda, int ka,
                                                           const float* B0, int64_t ldb0, int w0,
                                                           const float* B1, int64_t ldb1, int w1,
                                                           int64_t pe, float* part, int ncb) {
  __shared__ float sA[PT * LG];
  __shared__ float sB[PT * LG];
  const int s = blockIdx.x, cb = blockIdx.y;
  const int64_t r0 = (int64_t)s * GSLAB;
  load_cm<A_TS, GSLAB>(sA, LG, A, lda, r0, pe, ka);
  if (B0 != nullptr && cb == 0) {
    load_cm<false, GSLAB>(sB, LG, B0, ldb0, r0, pe, w0);
  } else {
    const int blk = cb - (B0 != nullptr ? 1 : 0);
    load_cm<true, GSLAB>(sB, LG, B1 + (int64_t)blk * PT * ldb1, ldb1, r0, pe, w1 - blk * PT);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int i = (wave >> 1) * 32 + l32, j = (wave & 1) * 32 + l32;
  f32x16 d;
  zero16(d);
#pragma unroll 8
  for (int st = 0; st < GSLAB / 2; ++st) {
    const int k = 2 * st + h;
    d = __builtin_amdgcn_mfma_f32_32x32x2f32(sA[i * LG + k], sB[j * LG + k], d, 0, 0, 0);
  }
  float* out = part + ((size_t)s * ncb + cb) * (PT * PT);
  const int jc = acc_col();
#pragma unroll
  for (int r = 0; r < 16; ++r) out[acc_row(r) * PT + jc] = d[r];
}

// G[cb * 4096 + e] = sum over s < nslab of part[(s * ncb + cb) * 4096 + e].
// A workgroup takes 32 consecutive elements; its eight 32-lane groups sum
// the slabs g, g + 8, g + 16, ... (all loads of a lane issued together), and
// the eight group sums are added in group order: a fixed association, so the
// result is deterministic, with one memory latency per element instead of
// nslab / 8.
constexpr int GR_E = 32, GR_G = PNT / GR_E;
__global__ __launch_bounds__(PNT) void gram_reduce_kernel(const float* part, int nslab, int ncb,
                                                          float* G) {
  __shared__ float acc_s[GR_G][GR_E];
  const int el = threadIdx.x % GR_E, g = threadIdx.x / GR_E;
  const int64_t idx = (int64_t)blockIdx.x * GR_E + el;   // over ncb * 4096
  const int64_t total = (int64_t)ncb * PT * PT;
  float acc = 0.0f;
  if (idx < total) {
    const int64_t cb = idx / (PT * PT), e = idx % (PT * PT);
    const float* p0 = part + cb * (PT * PT) + e;
    const int64_t stride = (int64_t)ncb * PT * PT;
    float v[8];
    for (int s0 = g; s0 < nslab; s0 += 8 * GR_G) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int sl = s0 + u * GR_G;
        v[u] = sl < nslab ? p0[(int64_t)sl * stride] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += v[u];
    }
  }
  acc_s[g][el] = acc;
  __syncthreads();
  if (g == 0 && idx < total) {
    float sum = acc_s[0][el];
#pragma unroll
    for (int q = 1; q < GR_G; ++q) sum += acc_s[q][el];
    G[idx] = sum;
  }
}

// Q2[r][:] = X_p[r][0:b] M (M b x b in ld b), r < pe, Q2 of ld 64 (columns >=
// b written as zero); X_p is the transposed row block XT (b x pe, ld ldx).
// When *flag is set (the first CholeskyQR pass collapsed) workgroup 0 runs
// the Householder fallback instead, which writes its reflectors into Q2 and
// R_new into P_top, and the other workgroups do nothing.
__global__ __launch_bounds__(PNT) void apply_m_kernel(const float* XT, int64_t ldx, int64_t pe,
                                                      int b, const float* M, float* Q2,
                                                      float* Ptop, int64_t ldr, const int* flag) {
  __shared__ float sX[PT * LT];
  __shared__ float sM[PT * TLD];
  if (*flag) {
    if (blockIdx.x == 0) panel_hh_fallback(Ptop, ldr, XT, ldx, pe, b, Q2, sX, sM);
    return;
  }
  const int64_t r0 = (int64_t)blockIdx.x * PT;
  load_cm<true, PT>(sX, LT, XT, ldx, r0, pe, b);
  load_rm(sM, M, b, b, b);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int m = (wave >> 1) * 32 + l32, n = (wave & 1) * 32 + l32;
  f32x16 d;
  zero16(d);
#pragma unroll 8
  for (int st = 0; st < 32; ++st) {
    const int k = 32 * h + st;
    d = __builtin_amdgcn_mfma_f32_32x32x2f32(sX[k * LT + m], sM[k * TLD + n], d, 0, 0, 0);
  }
  const int j = acc_col();
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t gr = r0 + acc_row(r);
    if (gr < pe) Q2[gr * PT + j] = d[r];
  }
}

// Panel update, one workgroup per (64-row tile, column block cb):
//   cb == 0:  Y[r][0:b] = Q2[r][:] N           (Y of ld ldy; RNE bf16 copies
//                                               into Yb, same ld, and into YbT
//                                               transposed, ld ldt, if given)
//   cb >= 1:  CT[c][r] -= (NW^T Q2^T)[c][r]    for the rows c of block cb - 1
//                                               of CT_rest (NW 64 x nr, ld ldnw)
// The transposed product puts consecutive r on consecutive lanes, so the
// read-modify-write of CT is coalesced.
__global__ __launch_bounds__(PNT) void panel_update_kernel(const float* Q2, int64_t pe, int b,
                                                           const float* N, float* Y, int64_t ldy,
                                                           bf16_t* Yb, bf16_t* YbT, int64_t ldt,
                                                           const float* NW, int64_t ldnw,
                                                           float* CT, int64_t ldc, int nr) {
  __shared__ float sQ[PT * LT];
  __shared__ float sM[PT * TLD];
  const int64_t r0 = (int64_t)blockIdx.x * PT;
  const int cb = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int mq = (wave >> 1) * 32 + l32, nq = (wave & 1) * 32 + l32;
  const int jc = acc_col();
  int w = b;
  // cb >= 1: the C entries this lane updates, loaded first so that their
  // latency overlaps the operand loads and the product
  const int64_t gr = r0 + jc;
  float* Cb = CT + (int64_t)(cb > 0 ? cb - 1 : 0) * PT * ldc + gr;
  float cur[16];
  if (cb > 0) {
    w = nr - (cb - 1) * PT;
    if (w > PT) w = PT;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int c = acc_row(r);
      cur[r] = (gr < pe && c < w) ? Cb[(int64_t)c * ldc] : 0.0f;
    }
  }
  load_cm<false, PT>(sQ, LT, Q2, PT, r0, pe, PT);
  if (cb == 0) load_rm(sM, N, b, b, b);
  else load_rm(sM, NW + (cb - 1) * PT, ldnw, PT, w);
  __syncthreads();
  f32x16 d;
  zero16(d);
  if (cb == 0) {
    // D[r][j] = sum_k Q2[r][k] N[k][j]
#pragma unroll 8
    for (int st = 0; st < 32; ++st) {
      const int k = 32 * h + st;
      d = __builtin_amdgcn_mfma_f32_32x32x2f32(sQ[k * LT + mq], sM[k * TLD + nq], d, 0, 0, 0);
    }
    if (jc < w) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t gr = r0 + acc_row(r);
        if (gr < pe) {
          Y[gr * ldy + jc] = d[r];
          if (Yb) Yb[gr * ldy + jc] = f32_to_bf16(d[r]);
        }
      }
    }
    if (YbT) {
      // the same product transposed, D[j][r] = sum_k N[k][j] Q2[r][k], so
      // consecutive r go to consecutive lanes and the rows of YbT are
      // written coalesced
      zero16(d);
#pragma unroll 8
      for (int st = 0; st < 32; ++st) {
        const int k = 32 * h + st;
        d = __builtin_amdgcn_mfma_f32_32x32x2f32(sM[k * TLD + mq], sQ[k * LT + nq], d, 0, 0, 0);
      }
      if (gr < pe) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = acc_row(r);
          if (j < w) YbT[(int64_t)j * ldt + gr] = f32_to_bf16(d[r]);
        }
      }
    }
  } else {
    // D[c][r] = sum_k NW[k][c] Q2[r][k]
#pragma unroll 8
    for (int st = 0; st < 32; ++st) {
      const int k = 32 * h + st;
      d = __builtin_amdgcn_mfma_f32_32x32x2f32(sM[k * TLD + mq], sQ[k * LT + nq], d, 0, 0, 0);
    }
    if (gr < pe) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = acc_row(r);
        if (c < w) Cb[(int64_t)c * ldc] = cur[r] - d[r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
int gram_slabs(int64_t pe) { return (int)cdiv(pe > 0 ? pe : 1, (int64_t)GSLAB); }

int launch_gram(hipStream_t s, const float* A, int64_t lda, int ka, bool a_ts, const float* B0,
                int64_t ldb0, int w0, const float* B1, int64_t ldb1, int w1, int64_t pe,
                float* part, float* G, int* ncb_out) {
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
  if (a_ts)
    hipLaunchKernelGGL(gram_partial_kernel<true>, dim3(ns, ncb), dim3(PNT), 0, s, A, lda, ka, B0,
                       ldb0, w0, B1, ldb1, w1, pe, part, ncb);
  else
    hipLaunchKernelGGL(gram_partial_kernel<false>, dim3(ns, ncb), dim3(PNT), 0, s, A, lda, ka, B0,
                       ldb0, w0, B1, ldb1, w1, pe, part, ncb);
  if (int rc = check_launch("gram_partial")) return rc;
  const int64_t total = (int64_t)ncb * PT * PT;
  hipLaunchKernelGGL(gram_reduce_kernel, dim3((unsigned)cdiv(total, (int64_t)GR_E)), dim3(PNT), 0,
                     s, part, ns, ncb, G);
  return check_launch("gram_reduce");
}

int launch_apply_m(hipStream_t s, const float* XT, int64_t ldx, int64_t pe, int b, const float* M,
                   float* Q2, float* Ptop, int64_t ldr, const int* flag) {
  if (b < 1 || b > PT) {
    set_error("apply_m: block size out of range");
    return IFK_ERR_INVALID;
  }
  // pe == 0 still launches one workgroup: a flagged panel needs the fallback
  hipLaunchKernelGGL(apply_m_kernel, dim3((unsigned)std::max<int64_t>(1, cdiv(pe, (int64_t)PT))),
                     dim3(PNT), 0, s, XT, ldx, pe, b, M, Q2, Ptop, ldr, flag);
  return check_launch("apply_m");
}

int launch_panel_update(hipStream_t s, const float* Q2, int64_t pe, int b, const float* N,
                        float* Y, int64_t ldy, bf16_t* Yb, bf16_t* YbT, int64_t ldt,
                        const float* NW, int64_t ldnw, float* CT, int64_t ldc, int nr) {
  if (pe <= 0) return IFK_OK;
  if (YbT && ldt < pe) {
    set_error("panel_update: transposed copy narrower than the panel");
    return IFK_ERR_INVALID;
  }
  const int nblk = nr > 0 ? (int)cdiv((int64_t)nr, (int64_t)PT) : 0;
  hipLaunchKernelGGL(panel_update_kernel, dim3((unsigned)cdiv(pe, (int64_t)PT), 1 + nblk),
                     dim3(PNT), 0, s, Q2, pe, b, N, Y, ldy, Yb, YbT, ldt, NW, ldnw, CT, ldc, nr);
  return check_launch("panel_update");
}

}  // namespace ifk
