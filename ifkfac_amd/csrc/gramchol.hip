// Fused fold + finalize by Gram matrix and blocked Cholesky (bf16 arithmetic).
//
// The damped factor of a factor update is the upper-triangular R with
//   R^T R = scale^2 (R_in^T R_in + X^T X) + damping I
// (activation_hooks.py:328-332 with triangular.py:246-307, 386-421: the QR of
// [scale R_in; scale X; sqrt(damping) I] with a positive diagonal, which is
// unique).  So R = scale * chol(A) with
//   A = P^T P + c^2 I,  P = [R_in; X],  c = sqrt(damping) / scale,
// and Q is never needed.  In bf16 arithmetic P is read as its RNE bf16
// rounding (what every MFMA operand of the fold gets), so the products of the
// Gram matrix are exact and only its fp32 accumulation rounds.
//
// Layout: the working matrix Aw (n x n fp32, row stride lda) keeps A's LOWER
// triangle, so that a column block below the diagonal (the panel of a
// Cholesky step and both operands of its Schur update) is a stack of
// contiguous rows: every large product reads K-contiguous operands on the
// direct-to-LDS kernel, with no transposes.  The factor is built as
// L = R^T / scale in place of A's lower triangle and cast to R at the end.
//
// Left-looking over GB-column blocks (1024; cholb factors one block).  Column
// block c (rows >= c0, the lower part) is
//   A_c = (P^T P)_c + c^2 I_cc - sum_{l < c} L_l L_{c,l}^T
// and step c factors it:
//   U_cc = chol(A_cc), M = U_cc^{-1}        (cholb, with M alongside)
//   L_cc = U_cc^T                            (into Aw)
//   L_rc = A_rc M                            (panel, rows below block c)
// The panel and the updates need fp32 accuracy from bf16 MFMA: operands are
// split as x = x_hi + x_lo (both RNE bf16), and a product is
// a_hi b_hi + a_hi b_lo + a_lo b_hi, formed as ONE product with K tripled by
// concatenating the halves along K:
//   panel:   [A_hi | A_lo | A_hi] . [M_hi | M_hi | M_lo]  (M given transposed)
//   updates: panel l is kept as LA = [L_hi | L_lo | L_hi] and LB = [L_lo |
//            L_hi | L_hi] at columns 3 GB l of two buffers, so the update of a
//            column by panels 0 .. m is one product over K = 3 GB (m + 1).
// The dropped lo.lo term and the roundings leave each product within about
// 2^-17 of |a||b|, far below the bf16 rounding of the stored factor.
//
// Look-ahead: the calling stream runs the chain of steps (latency-bound:
// cholb is a chain of 64-column launches); the helper stream prepares column
// c + 2 -- its Gram columns, the damping, and the updates by panels 0 .. c --
// while step c + 1 runs, so the Gram matrix (p n^2 flops for its lower part)
// and most of the updates (n^3 in all, split) are done beside the chain.
// Step c itself applies only the update by panel c - 1.
//
// Pivot test: a pivot below the tolerance pivot_tol (GRAM_PIVOT_TOL, 1e-3, by
// default for the factor update; the streaming fold's caller passes its own)
// times the Gram diagonal of its column
// (A's diagonal before any update) means that column is nearly a combination
// of the ones before it (cancellation of more than 1 - pivot_tol in the Schur
// complement): the rounding of the Gram matrix and of the updates, about
// 2^-17 of that diagonal, would then be a visible part of the pivot.  The
// call then reports status 2, and the caller recomputes the factor by the
// TPQRT fold (linalg.hip), which never forms A.  Non-finite input raises the
// same flag (NaN pivots fail the test).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <mutex>

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

namespace {

constexpr int64_t GB = 1024;          // Cholesky block (cholb supports up to 1024)

// ---------------------------------------------------------------------------
// Kernels.  Every one takes a batch of same-shaped problems: entry b of a
// launch is blockIdx.y (blockIdx.z for the 2-D tiled ones), at the given
// element strides from each pointer.
// ---------------------------------------------------------------------------

// dst (cols x rows, bf16, row stride ldd) = src^T for a rows x cols block of
// fp32 or bf16 src; with upper set, entries of src below its diagonal are
// taken as zero.  64 x 64 LDS tile: fp32 rows read as float4 (vec_in: src
// 16-byte aligned, lds a multiple of 4), the output written as bf16 pairs
// (pairs_out: dst 4-byte aligned, ldd even); element-wise otherwise.  With
// dst2 set, each value x is split as x = hi + lo (both RNE bf16) and the rows
// of dst get three segments of rows elements [hi | lo | hi], those of dst2
// [hi | hi | lo]: K-concatenated operands whose product is
// hi hi^T + lo hi^T + hi lo^T, x x^T to about 2^-17.
template <int DT>
__global__ __launch_bounds__(256) void transpose_to_bf16_kernel(const void* src, int64_t lds,
                                                                int64_t rows, int64_t cols,
                                                                bf16_t* dst, int64_t ldd,
                                                                int upper, int vec_in,
                                                                int pairs_out, bf16_t* dst2) {
  __shared__ float tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int t = threadIdx.x;
  typedef typename Elem<DT>::T ST;
  const ST* S = (const ST*)src;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int rl = (t >> 4) + 16 * q, cl = (t & 15) * 4;
    const int64_t r = r0 + rl, c = c0 + cl;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (r < rows) {
      if (DT == DT_F32 && vec_in && c + 3 < cols) {
        const float4 x = *reinterpret_cast<const float4*>((const float*)src + r * lds + c);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
      } else {
        for (int u = 0; u < 4; ++u)
          if (c + u < cols) v[u] = Elem<DT>::load(S + r * lds + c + u);
      }
      if (upper)
        for (int u = 0; u < 4; ++u)
          if (r > c + u) v[u] = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) tile[rl][cl + u] = v[u];
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int idx = t + 256 * q, cl = idx >> 5, rp = (idx & 31) * 2;
    const int64_t c = c0 + cl, r = r0 + rp;
    if (c >= cols || r >= rows) continue;
    bf16_t* g = dst + c * ldd + r;
    if (dst2) {
      // split: x = hi + lo (both RNE bf16); dst gets [hi | lo | hi] and
      // dst2 [hi | hi | lo] in three segments of rows elements along its rows
      bf16_t* g2 = dst2 + c * ldd + r;
      for (int u = 0; u < 2 && r + u < rows; ++u) {
        const float x = tile[rp + u][cl];
        const bf16_t hi = f32_to_bf16(x);
        const bf16_t lo = f32_to_bf16(x - bf16_to_f32(hi));
        g[u] = hi;
        g[rows + u] = lo;
        g[2 * rows + u] = hi;
        g2[u] = hi;
        g2[rows + u] = hi;
        g2[2 * rows + u] = lo;
      }
    } else if (pairs_out && r + 1 < rows) {
      *reinterpret_cast<uint32_t*>(g) = pack_bf16x2(tile[rp][cl], tile[rp + 1][cl]);
    } else {
      g[0] = f32_to_bf16(tile[rp][cl]);
      if (r + 1 < rows) g[1] = f32_to_bf16(tile[rp + 1][cl]);
    }
  }
}

// Split rows x cols fp32 into nseg consecutive bf16 segments per row,
// dst[r][s cols + c] = lo(x) if bit s of lo_mask else hi(x), hi = RNE(x),
// lo = RNE(x - hi), and the same into dst2 (ldd2, lo_mask2) when given.
// Four columns per thread (cols % 4 == 0, 16-byte rows).
struct SegStrides {
  int64_t src = 0, dst = 0, dst2 = 0;
};
__global__ __launch_bounds__(256) void split_seg_kernel(const float* src, int64_t lds,
                                                        int64_t rows, int64_t cols, bf16_t* dst,
                                                        int64_t ldd, int nseg, int lo_mask,
                                                        bf16_t* dst2, int64_t ldd2, int lo_mask2,
                                                        SegStrides bs) {
  {
    const int64_t b = blockIdx.y;
    src += b * bs.src;
    dst += b * bs.dst;
    if (dst2) dst2 += b * bs.dst2;
  }
  const int64_t c4 = cols >> 2;
  const int64_t total = rows * c4;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / c4, c = (e - r * c4) * 4;
    const float4 x = *reinterpret_cast<const float4*>(src + r * lds + c);
    const float v[4] = {x.x, x.y, x.z, x.w};
    bf16_t h[4], l[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      h[u] = f32_to_bf16(v[u]);
      l[u] = f32_to_bf16(v[u] - bf16_to_f32(h[u]));
    }
    const uint2 hw = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16),
                                (uint32_t)h[2] | ((uint32_t)h[3] << 16));
    const uint2 lw = make_uint2((uint32_t)l[0] | ((uint32_t)l[1] << 16),
                                (uint32_t)l[2] | ((uint32_t)l[3] << 16));
    bf16_t* d = dst + r * ldd + c;
    for (int s = 0; s < nseg; ++s)
      *reinterpret_cast<uint2*>(d + s * cols) = ((lo_mask >> s) & 1) ? lw : hw;
    if (dst2) {
      bf16_t* d2 = dst2 + r * ldd2 + c;
      for (int s = 0; s < nseg; ++s)
        *reinterpret_cast<uint2*>(d2 + s * cols) = ((lo_mask2 >> s) & 1) ? lw : hw;
    }
  }
}

// G (n x n, ldg) = the symmetric matrix whose lower triangle is A's (lda):
// G_ij = A_max(i,j),min(i,j).  Tile (tr, tc) of G reads A's tile
// (max, min) once through LDS.
__global__ __launch_bounds__(256) void sym_from_lower_kernel(const float* A, int64_t lda,
                                                             int64_t n, float* G, int64_t ldg,
                                                             int64_t sa, int64_t sg) {
  __shared__ float tile[32][33];
  A += (int64_t)blockIdx.z * sa;
  G += (int64_t)blockIdx.z * sg;
  const int tr = blockIdx.y, tc = blockIdx.x;
  const int ar = tr > tc ? tr : tc, ac = tr > tc ? tc : tr;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = (int64_t)ar * 32 + k, c = (int64_t)ac * 32 + tx;
    tile[k][tx] = (r < n && c < n) ? A[r * lda + c] : 0.0f;
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = (int64_t)tr * 32 + k, c = (int64_t)tc * 32 + tx;
    if (r >= n || c >= n) continue;
    float v;
    if (tr > tc) v = tile[k][tx];
    else if (tr < tc) v = tile[tx][k];
    else v = (k >= tx) ? tile[k][tx] : tile[tx][k];
    G[r * ldg + c] = v;
  }
}

// out (odt, n x n, ldo) = scale * L^T for the lower-triangular L (ldl):
// out_ij = scale L_ji for j >= i, 0 below the diagonal; finite[b] = 0 when
// any stored value is not finite.
template <int ODT>
__global__ __launch_bounds__(256) void cast_lower_t_kernel(const float* L, int64_t ldl, int64_t n,
                                                           float scale, void* out, int64_t ldo,
                                                           int* finite, int64_t sl,
                                                           int64_t so) {
  __shared__ float tile[32][33];
  const int64_t b = blockIdx.z;
  L += b * sl;
  finite += b;
  const int tr = blockIdx.y, tc = blockIdx.x;   // output tile
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  typedef typename Elem<ODT>::T OT;
  OT* O = (OT*)out + b * so;
  if (tr > tc) {
    for (int k = ty; k < 32; k += 8) {
      const int64_t r = (int64_t)tr * 32 + k, c = (int64_t)tc * 32 + tx;
      if (r < n && c < n) Elem<ODT>::store(O + r * ldo + c, 0.0f);
    }
    return;
  }
  // L's tile (tc, tr) holds the output tile transposed
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = (int64_t)tc * 32 + k, c = (int64_t)tr * 32 + tx;
    tile[k][tx] = (r < n && c < n) ? L[r * ldl + c] : 0.0f;
  }
  __syncthreads();
  bool bad = false;
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = (int64_t)tr * 32 + k, c = (int64_t)tc * 32 + tx;
    if (r >= n || c >= n) continue;
    const float v = (c >= r) ? scale * tile[tx][k] : 0.0f;
    if (!isfinite(v)) bad = true;
    Elem<ODT>::store(O + r * ldo + c, v);
  }
  if (bad) *finite = 0;
}

// A_ii += v and dref_i = A_ii (after the addition), i < n
__global__ void add_diag_ref_kernel(float* A, int64_t lda, int64_t n, float v, float* dref,
                                    int64_t sa, int64_t sd) {
  A += (int64_t)blockIdx.y * sa;
  dref += (int64_t)blockIdx.y * sd;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float d = A[i * lda + i] + v;
    A[i * lda + i] = d;
    dref[i] = d;
  }
}

// Sum of squares of a Gram column block's lower part (rows x W at A, row
// stride lda a multiple of 4, A 16-byte aligned, W <= 1024; the block's
// diagonal at its top, entries above it ignored), off-diagonal entries
// counted twice (they stand for both triangles): workgroup g takes rows g,
// g + FROB_WG, ... with four consecutive columns per thread (one float4 when
// all four lie in the block) and writes one partial to part[g], so the
// result does not depend on scheduling.
constexpr int FROB_WG = 1024;
__global__ __launch_bounds__(256) void gram_frob_kernel(const float* A, int64_t lda, int64_t rows,
                                                        int64_t W, int64_t r_off, float* part,
                                                        int64_t sa, int64_t sp) {
  __shared__ float red[4];
  A += (int64_t)blockIdx.y * sa;
  part += (int64_t)blockIdx.y * sp;
  float acc = 0.0f;
  const int64_t c = (int64_t)threadIdx.x * 4;
  if (c < W) {
    for (int64_t r = blockIdx.x; r < rows; r += FROB_WG) {
      float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (c + 3 < W) {
        const float4 v = *reinterpret_cast<const float4*>(A + r * lda + c);
        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
      } else {
        for (int u = 0; c + u < W; ++u) x[u] = A[r * lda + c + u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t cc = c + u;
        if (cc < W && cc <= r + r_off) acc = fmaf(cc == r + r_off ? x[u] : 2.0f * x[u], x[u], acc);
      }
    }
  }
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// kb[b] = sqrt(1 + scale^2 sqrt(sum of entry b's count partials) / damping):
// with E = scale^2 P^T P, kappa_2(R)^2 = kappa(E + damping I)
// <= 1 + ||E||_2 / damping <= 1 + ||E||_F / damping.  Infinite without
// damping.  256 threads per entry: strided sums in a fixed order, then a
// fixed tree.
__global__ __launch_bounds__(256) void kappa_bound_kernel(const float* part, int count,
                                                          float scale, float damping, float* kb) {
  __shared__ double red[256];
  part += (int64_t)blockIdx.x * count;
  double ss = 0.0;
  for (int i = threadIdx.x; i < count; i += 256) ss += (double)part[i];
  red[threadIdx.x] = ss;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double e = (double)scale * (double)scale * sqrt(red[0]);
    kb[blockIdx.x] = damping > 0.0f ? (float)sqrt(1.0 + e / (double)damping) : INFINITY;
  }
}

// status[b] = 2 where flag[b] is set (flags at int stride fs)
__global__ void status_merge_batch_kernel(int* status, const int* flag, int64_t fs, int batch) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < batch && flag[b * fs] != 0) status[b] = 2;
}

// MT3 (W x 3 GB bf16, row stride ld3) = [hi(M^T) | hi(M^T) | lo(M^T)] for the
// upper-triangular M (W x W, ldm; entries below its diagonal read as zero),
// hi = RNE(x), lo = RNE(x - hi); batch entry blockIdx.z at the strides sm,
// s3.  32 x 32 tiles through LDS.
__global__ __launch_bounds__(256) void mt3_kernel(const float* M, int64_t ldm, int64_t W,
                                                  bf16_t* MT3, int64_t ld3, int64_t sm,
                                                  int64_t s3) {
  __shared__ float tile[32][33];
  M += (int64_t)blockIdx.z * sm;
  MT3 += (int64_t)blockIdx.z * s3;
  const int tr = blockIdx.y, tc = blockIdx.x;   // output tile (row block of M^T)
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  // M's tile (tc, tr) is the output tile transposed
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = (int64_t)tc * 32 + k, c = (int64_t)tr * 32 + tx;
    tile[k][tx] = (r < W && c < W && r <= c) ? M[r * ldm + c] : 0.0f;
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = (int64_t)tr * 32 + k, c = (int64_t)tc * 32 + tx;
    if (r >= W || c >= W) continue;
    const float x = tile[tx][k];
    const bf16_t hi = f32_to_bf16(x), lo = f32_to_bf16(x - bf16_to_f32(hi));
    bf16_t* o = MT3 + r * ld3 + c;
    o[0] = hi;
    o[GB] = hi;
    o[2 * GB] = lo;
  }
}

// Diagonal block of the inverse: Z = alpha M on and above the diagonal (zero
// below), its RNE bf16 copy Zb and the transposed copy ZT (zero above), a W x
// W block of each; batch entry blockIdx.z at the element strides sm, sz, sb.
// 32 x 32 tiles through LDS, so the transposed copy is written by rows too.
__global__ __launch_bounds__(256) void diag_inverse_kernel(const float* M, int64_t ldm, int64_t W,
                                                           float alpha, float* Z, int64_t ldz,
                                                           bf16_t* Zb, bf16_t* ZT, int64_t ldb,
                                                           int64_t sm, int64_t sz, int64_t sb) {
  __shared__ float tile[32][33];
  const int64_t e = blockIdx.z;
  M += e * sm;
  Z += e * sz;
  Zb += e * sb;
  ZT += e * sb;
  const int tr = blockIdx.y, tc = blockIdx.x;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = (int64_t)tr * 32 + k, c = (int64_t)tc * 32 + tx;
    float v = 0.0f;
    if (r < W && c < W) {
      if (c >= r) v = alpha * M[r * ldm + c];
      Z[r * ldz + c] = v;
      Zb[r * ldb + c] = f32_to_bf16(v);
    }
    tile[k][tx] = v;
  }
  __syncthreads();
  // ZT's tile (tc, tr): ZT[r][c] = Z[c][r]
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = (int64_t)tc * 32 + k, c = (int64_t)tr * 32 + tx;
    if (r < W && c < W) ZT[r * ldb + c] = f32_to_bf16(tile[tx][k]);
  }
}

unsigned grid_of(int64_t work, int64_t cap = 2048) {
  int64_t g = cdiv(work, 256);
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

int transpose_to_bf16(hipStream_t s, const void* src, int sdt, int64_t lds, int64_t rows,
                      int64_t cols, bf16_t* dst, int64_t ldd, bool upper,
                      bf16_t* dst2 = nullptr) {
  if (rows * cols == 0) return IFK_OK;
  if (cdiv(rows, 64) > 65535) {
    set_error("fold_finalize_gram: too many rows to transpose");
    return IFK_ERR_INVALID;
  }
  const int vec_in = (((uintptr_t)src & 15) == 0) && (lds % 4 == 0);
  const int pairs_out = (((uintptr_t)dst & 3) == 0) && (ldd % 2 == 0);
  const dim3 grid((unsigned)cdiv(cols, 64), (unsigned)cdiv(rows, 64));
  if (sdt == DT_F32)
    hipLaunchKernelGGL(transpose_to_bf16_kernel<DT_F32>, grid, dim3(256), 0, s, src, lds, rows,
                       cols, dst, ldd, upper ? 1 : 0, vec_in, pairs_out, dst2);
  else
    hipLaunchKernelGGL(transpose_to_bf16_kernel<DT_BF16>, grid, dim3(256), 0, s, src, lds, rows,
                       cols, dst, ldd, upper ? 1 : 0, 0, pairs_out, dst2);
  return check_launch("transpose_to_bf16");
}

int split_seg(hipStream_t s, int batch, const float* src, int64_t lds, int64_t rows, int64_t cols,
              bf16_t* dst, int64_t ldd, int nseg, int lo_mask, SegStrides bs,
              bf16_t* dst2 = nullptr, int64_t ldd2 = 0, int lo_mask2 = 0) {
  if (rows * cols == 0) return IFK_OK;
  hipLaunchKernelGGL(split_seg_kernel, dim3(grid_of(rows * cols / 4, 1024), (unsigned)batch),
                     dim3(256), 0, s, src, lds, rows, cols, dst, ldd, nseg, lo_mask, dst2, ldd2,
                     lo_mask2, bs);
  return check_launch("split_seg");
}

int sym_from_lower(hipStream_t s, int batch, const float* A, int64_t lda, int64_t n, float* G,
                   int64_t ldg, int64_t sa, int64_t sg) {
  const dim3 grid((unsigned)cdiv(n, 32), (unsigned)cdiv(n, 32), (unsigned)batch);
  hipLaunchKernelGGL(sym_from_lower_kernel, grid, dim3(256), 0, s, A, lda, n, G, ldg, sa, sg);
  return check_launch("sym_from_lower");
}

int cast_lower_t(hipStream_t s, int batch, const float* L, int64_t ldl, int64_t n, float scale,
                 void* out, int odt, int64_t ldo, int* finite, int64_t sl, int64_t so) {
  if (cdiv(n, 32) > 65535) {
    set_error("fold_finalize_gram: factor too large");
    return IFK_ERR_INVALID;
  }
  const dim3 grid((unsigned)cdiv(n, 32), (unsigned)cdiv(n, 32), (unsigned)batch);
  if (odt == DT_F32)
    hipLaunchKernelGGL(cast_lower_t_kernel<DT_F32>, grid, dim3(256), 0, s, L, ldl, n, scale, out,
                       ldo, finite, sl, so);
  else
    hipLaunchKernelGGL(cast_lower_t_kernel<DT_BF16>, grid, dim3(256), 0, s, L, ldl, n, scale, out,
                       ldo, finite, sl, so);
  return check_launch("cast_lower_t");
}

// ---------------------------------------------------------------------------
// Workspace (every buffer once per batch entry, at the stride s*)
// ---------------------------------------------------------------------------
// Workgroup caps of the helper streams' products: the chain's launches
// (cholb's diagonal workgroup, the band products) must find CUs free while
// the Gram columns and the panel work run beside them.
constexpr int GRAM_MAX_WGS = 128;
constexpr int REST_MAX_WGS = 192;

struct GramWs {
  int64_t B;          // batch entries
  int64_t ldk;        // row stride of PT and PB (K rows rounded up to 8; the pad is zero)
  int64_t kr;         // K offset of the chunk's rows: r_in, or 3 r_in with the split
  int64_t lda;        // row stride of Aw
  int64_t ldl;        // row stride of LA / LB: 3 GB per panel
  bf16_t* PT;         // P^T in bf16, n x ldk: the A operand of the Gram products
  bf16_t* PB;         // their B operand: PT itself, or with the split running
                      // factor the K segments [R_hi | R_hi | R_lo | X] against
                      // PT's [R_hi | R_lo | R_hi | X]
  float* Aw;          // working matrix / factor (lower), n x lda
  float* dref;        // Gram diagonal (+ c^2), n
  float* G;           // symmetrised diagonal block, GB x GB; then M^T
  float* U;           // U_kk, GB x GB
  float* Mh;          // U_kk^{-1} of every block k, at k GB^2 (nb GB x GB blocks)
  float* Zd;          // cholb's 64 x 64 diagonal inverses, GB x 64
  bf16_t* MT3[2];     // [M^T_hi | M^T_hi | M^T_lo], GB x 3 GB, by step parity
  bf16_t* ASb;        // [A_hi | A_lo | A_hi] of the band block, GB x 3 GB
  bf16_t* LSb;        // [L_hi | L_lo | L_hi | L_hi] of the band block, GB x 4 GB
  bf16_t* AS2;        // [A_hi | A_lo | A_hi] of the rest of a panel, n x 3 GB
  bf16_t* LA;         // panel l at columns 3 GB l: [L_hi | L_lo | L_hi], n x ldl
  bf16_t* LB;         // panel l at columns 3 GB l: [L_lo | L_hi | L_hi], n x ldl
  int* flag;          // one per entry, at int stride FLAG_S
  float* frob;        // per entry and Gram column, FROB_WG partial sums of squares (column 0's
                      // diagonal block in the extra set nb, its rows below in set 0)
  bf16_t* Tinv;       // the inverse's doubling levels: n^2 / 4 bf16 (one entry at a time)
  int64_t sPT, sAw, sdref, sGB, sMh, sZd, sMT3, sLSb, sAS2, sL, sfrob;
  SplitScratch sp, sp2, sp3;   // split-K partials of the three streams
  float tol;                   // relative pivot threshold of the pivot test
};
constexpr int64_t FLAG_S = 64;   // ints between two entries' flags (separate cache lines)

void plan_gram(Arena& a, int64_t B, int64_t p, int64_t r_in, int64_t n, GramWs& w,
               bool inv = false, bool split_r = false) {
  const int64_t nb = cdiv(n, GB);
  const bool two = split_r && r_in > 0;
  const int64_t pe = (two ? 3 * r_in : r_in) + p;   // K extent of the Gram products
  w.B = B;
  w.kr = two ? 3 * r_in : r_in;
  w.ldk = (int64_t)align_up((size_t)std::max<int64_t>(pe, 1), 8);
  w.lda = (int64_t)align_up((size_t)n, 64);
  w.ldl = 3 * GB * std::max<int64_t>(nb - 1, 1);
  const bool multi = nb > 1;
  const int64_t big = multi ? n : 1;
  // strides rounded to 64 elements: every entry's buffers stay 256-byte aligned
  auto al = [](int64_t e) { return (int64_t)align_up((size_t)e, 64); };
  w.sPT = al(n * w.ldk);
  w.sAw = al(n * w.lda);
  w.sdref = al(n);
  w.sGB = GB * GB;
  w.sMh = nb * GB * GB;
  w.sZd = (GB / 64) * 64 * 64;
  w.sMT3 = multi ? GB * 3 * GB : 64;
  w.sLSb = multi ? GB * 4 * GB : 64;
  w.sAS2 = al(big * 3 * GB);
  w.sL = al(big * w.ldl);
  w.sfrob = (nb + 1) * FROB_WG;   // + the diagonal block of column 0, kept apart
  w.PT = a.take<bf16_t>((size_t)(B * w.sPT));
  w.PB = two ? a.take<bf16_t>((size_t)(B * w.sPT)) : w.PT;
  w.Aw = a.take<float>((size_t)(B * w.sAw));
  w.dref = a.take<float>((size_t)(B * w.sdref));
  w.G = a.take<float>((size_t)(B * w.sGB));
  w.U = a.take<float>((size_t)(B * w.sGB));
  w.Mh = a.take<float>((size_t)(B * w.sMh));
  w.Tinv = inv ? a.take<bf16_t>((size_t)(n * n / 4 + 64)) : nullptr;
  w.Zd = a.take<float>((size_t)(B * w.sZd));
  for (int i = 0; i < 2; ++i) w.MT3[i] = a.take<bf16_t>((size_t)(B * w.sMT3));
  w.ASb = a.take<bf16_t>((size_t)(B * w.sMT3));
  w.LSb = a.take<bf16_t>((size_t)(B * w.sLSb));
  w.AS2 = a.take<bf16_t>((size_t)(B * w.sAS2));
  w.LA = a.take<bf16_t>((size_t)(B * w.sL));
  w.LB = a.take<bf16_t>((size_t)(B * w.sL));
  w.flag = a.take<int>((size_t)(B * FLAG_S));
  w.frob = a.take<float>((size_t)(B * w.sfrob));
  // split-K and stream-K partials of the products with one block column of
  // output: the chain's band products (GB x GB, K = 3 GB), the helper's
  // panel and column updates (up to n x GB, K up to 3 GB (nb - 1)) and the
  // Gram columns (n x GB, K = pe).  Stream-K needs are per entry times B, so
  // a batch takes the grid a batch of one takes (the same bits).
  const int64_t kmax2 = 3 * GB * std::max<int64_t>(nb - 1, 1);
  w.sp.floats = std::max((size_t)(B * std::min<int64_t>(n, 8 * GB) * GB * 2),
                         (size_t)B * gemm_scratch_floats(GB, GB, 3 * GB, 1));
  w.sp.p = a.take<float>(w.sp.floats);
  w.sp2.floats = std::max((size_t)(B * std::min<int64_t>(n, 16 * GB) * GB * 2),
                          (size_t)B * gemm_scratch_floats(n, GB, kmax2, 1, REST_MAX_WGS));
  w.sp2.p = a.take<float>(w.sp2.floats);
  w.sp3.floats = std::max((size_t)(B * std::min<int64_t>(n, 16 * GB) * GB * 2),
                          (size_t)B * gemm_scratch_floats(n, GB, std::max<int64_t>(pe, 1), 1,
                                                          GRAM_MAX_WGS));
  w.sp3.p = a.take<float>(w.sp3.floats);
}

// Gram column c >= GRAM_LEAD starts only when helper step c - GRAM_LEAD is
// done.  Unthrottled, the Gram stream runs far ahead of the chain and holds
// its CUs for the whole first half of the factorisation, while the helper's
// panel work -- which the chain waits for -- gets what is left; throttled,
// the Gram columns stay a few blocks ahead of where the helper needs them
// (helper step k waits for column k + 2, so the lead must be at least 3).
constexpr int64_t GRAM_LEAD = 4;
static_assert(GRAM_LEAD >= 3, "helper step k must find column k + 2 enqueued");

struct Blk {
  int64_t r0, r1;   // rows / columns of block k
};
inline Blk blk(int64_t k, int64_t n) { return Blk{k * GB, std::min<int64_t>(k * GB + GB, n)}; }

// Gram column c of A (rows >= c0, lower part) with c^2 on its diagonal and
// the pivot test's reference diagonal taken there, for every entry.
int gram_column(hipStream_t s, GramWs& w, int64_t n, int64_t c, float c2, bool have_rows,
                int max_wgs) {
  const Blk b = blk(c, n);
  const int64_t W = b.r1 - b.r0, rows = n - b.r0;
  const int B = (int)w.B;
  float* Ac = w.Aw + b.r0 * w.lda + b.r0;
  if (have_rows) {
    RC(gemm(s, MATH_BF16, rows, W, w.ldk, 1.0f,
            A_n(w.PT + b.r0 * w.ldk, DT_BF16, w.ldk, TRI_NONE, w.sPT),
            B_t(w.PB + b.r0 * w.ldk, DT_BF16, w.ldk, TRI_NONE, w.sPT), 0.0f,
            per_entry(lower_part(out_f32(Ac, w.lda, w.sAw))), B, w.sp3, max_wgs));
  } else {
    for (int e = 0; e < B; ++e) RC(launch_zero(s, Ac + e * w.sAw, w.lda, rows, W));
  }
  hipLaunchKernelGGL(gram_frob_kernel, dim3(FROB_WG, (unsigned)B), dim3(256), 0, s, Ac, w.lda,
                     rows, W, (int64_t)0, w.frob + c * FROB_WG, w.sAw, w.sfrob);
  RC(check_launch("gram_frob"));
  hipLaunchKernelGGL(add_diag_ref_kernel, dim3(grid_of(W, 64), (unsigned)B), dim3(256), 0, s, Ac,
                     w.lda, W, c2, w.dref + b.r0, w.sAw, w.sdref);
  return check_launch("add_diag_ref");
}

// Gram column 0 in two parts, so that the chain can start on the first: its
// diagonal block (with c^2 and the reference diagonal), and its rows below.
int gram_column0_diag(hipStream_t s, GramWs& w, int64_t n, float c2, bool have_rows,
                      int max_wgs) {
  const Blk b = blk(0, n);
  const int64_t W = b.r1 - b.r0;
  const int B = (int)w.B;
  float* Ac = w.Aw;
  if (have_rows) {
    RC(gemm(s, MATH_BF16, W, W, w.ldk, 1.0f, A_n(w.PT, DT_BF16, w.ldk, TRI_NONE, w.sPT),
            B_t(w.PB, DT_BF16, w.ldk, TRI_NONE, w.sPT), 0.0f,
            per_entry(lower_part(out_f32(Ac, w.lda, w.sAw))), B, w.sp3, max_wgs));
  } else {
    for (int e = 0; e < B; ++e) RC(launch_zero(s, Ac + e * w.sAw, w.lda, W, W));
  }
  const int64_t nb = cdiv(n, GB);
  hipLaunchKernelGGL(gram_frob_kernel, dim3(FROB_WG, (unsigned)B), dim3(256), 0, s, Ac, w.lda, W,
                     W, (int64_t)0, w.frob + nb * FROB_WG, w.sAw, w.sfrob);
  RC(check_launch("gram_frob"));
  hipLaunchKernelGGL(add_diag_ref_kernel, dim3(grid_of(W, 64), (unsigned)B), dim3(256), 0, s, Ac,
                     w.lda, W, c2, w.dref, w.sAw, w.sdref);
  return check_launch("add_diag_ref");
}

int gram_column0_rest(hipStream_t s, GramWs& w, int64_t n, bool have_rows, int max_wgs) {
  const Blk b = blk(0, n);
  const int64_t W = b.r1 - b.r0, rows = n - W;
  const int B = (int)w.B;
  float* Ac = w.Aw + W * w.lda;
  if (rows <= 0) {
    // one block: the set of the rows below stays empty
    hipLaunchKernelGGL(gram_frob_kernel, dim3(FROB_WG, (unsigned)B), dim3(256), 0, s, w.Aw, w.lda,
                       (int64_t)0, W, W, w.frob, w.sAw, w.sfrob);
    return check_launch("gram_frob");
  }
  if (have_rows) {
    RC(gemm(s, MATH_BF16, rows, W, w.ldk, 1.0f,
            A_n(w.PT + W * w.ldk, DT_BF16, w.ldk, TRI_NONE, w.sPT),
            B_t(w.PB, DT_BF16, w.ldk, TRI_NONE, w.sPT), 0.0f,
            per_entry(out_f32(Ac, w.lda, w.sAw)), B, w.sp3, max_wgs));
  } else {
    for (int e = 0; e < B; ++e) RC(launch_zero(s, Ac + e * w.sAw, w.lda, rows, W));
  }
  hipLaunchKernelGGL(gram_frob_kernel, dim3(FROB_WG, (unsigned)B), dim3(256), 0, s, Ac, w.lda,
                     rows, W, W, w.frob, w.sAw, w.sfrob);
  return check_launch("gram_frob");
}

// Chain, part 1 of step k: L_kk = chol(A_kk)^T and M = U_kk^{-1}.
int chain_factor(hipStream_t s, GramWs& w, int64_t n, int64_t k) {
  const Blk b = blk(k, n);
  const int64_t W = b.r1 - b.r0;
  const int B = (int)w.B;
  float* Akk = w.Aw + b.r0 * w.lda + b.r0;
  RC(sym_from_lower(s, B, Akk, w.lda, W, w.G, GB, w.sAw, w.sGB));
  CholbStrides cs;
  cs.a = w.sGB; cs.u = w.sGB; cs.zd = w.sZd; cs.dref = w.sdref; cs.m = w.sMh; cs.flag = FLAG_S;
  float* Mk = w.Mh + k * GB * GB;
  // (cholb leaves M's blocks below the diagonal unset; their readers take
  // the upper triangle only)
  RC(launch_cholb(s, w.G, GB, (int)W, w.U, GB, w.Zd, w.dref + b.r0, w.tol, w.flag, Mk, GB,
                  true, B, cs));
  return launch_transpose_cast(s, w.U, GB, W, W, Akk, DT_F32, w.lda, B, w.sGB, w.sAw);
}

// ASb = [A_hi | A_lo | A_hi] of block (k + 1, k), the band product's operand.
int split_band(hipStream_t s, GramWs& w, int64_t n, int64_t k) {
  const Blk b = blk(k, n), b1 = blk(k + 1, n);
  SegStrides a3;
  a3.src = w.sAw; a3.dst = w.sMT3;
  return split_seg(s, (int)w.B, w.Aw + b1.r0 * w.lda + b.r0, w.lda, b1.r1 - b1.r0, b.r1 - b.r0,
                   w.ASb, 3 * GB, 3, 0b010, a3);
}

// Chain, part 2 of step k (block k + 1 exists): M^T split into MT3[k % 2];
// the band L_{k+1,k} = A_{k+1,k} M; the next diagonal block's update
// A_{k+1,k+1} -= L_{k+1,k} L_{k+1,k}^T.
int chain_band(hipStream_t s, GramWs& w, int64_t n, int64_t k) {
  const Blk b = blk(k, n), b1 = blk(k + 1, n);
  const int64_t W = b.r1 - b.r0, W1 = b1.r1 - b1.r0;   // W == GB here
  const int B = (int)w.B;
  bf16_t* MT3 = w.MT3[k & 1];
  const dim3 tg((unsigned)cdiv(W, 32), (unsigned)cdiv(W, 32), (unsigned)B);
  hipLaunchKernelGGL(mt3_kernel, tg, dim3(256), 0, s, w.Mh + k * GB * GB, GB, W, MT3, 3 * GB,
                     w.sMh, w.sMT3);
  RC(check_launch("mt3"));
  float* Ab = w.Aw + b1.r0 * w.lda + b.r0;   // block (k + 1, k)
  // the band's split copy: helper step k - 1 made it (as soon as the block
  // was final), step 0 makes its own
  if (k == 0) RC(split_band(s, w, n, 0));
  RC(gemm(s, MATH_BF16, W1, W, 3 * W, 1.0f, A_n(w.ASb, DT_BF16, 3 * GB, TRI_NONE, w.sMT3),
          B_t(MT3, DT_BF16, 3 * GB, TRI_NONE, w.sMT3), 0.0f, per_entry(out_f32(Ab, w.lda, w.sAw)), B,
          w.sp));
  SegStrides l4;
  l4.src = w.sAw; l4.dst = w.sLSb;
  RC(split_seg(s, B, Ab, w.lda, W1, W, w.LSb, 4 * GB, 4, 0b0010, l4));
  float* A11 = w.Aw + b1.r0 * w.lda + b1.r0;
  return gemm(s, MATH_BF16, W1, W1, 3 * W, -1.0f, A_n(w.LSb, DT_BF16, 4 * GB, TRI_NONE, w.sLSb),
              B_t(w.LSb + GB, DT_BF16, 4 * GB, TRI_NONE, w.sLSb), 1.0f,
              per_entry(lower_part(out_f32(A11, w.lda, w.sAw))), B, w.sp);
}

// Helper work of step k (blocks k + 2 .. exist): the rest of panel k,
// L_{>k+1,k} = A_{>k+1,k} M (in place); panel k's split copies (rows > k);
// column k + 1's rows > k + 1 updated by panel k; column k + 2 updated by
// panels 0 .. k (after its Gram column, event gev_k2).
int helper_step(hipStream_t s, GramWs& w, int64_t n, int64_t k, hipEvent_t gev_k2,
                hipEvent_t gev_k1, int max_wgs) {
  const Blk b = blk(k, n), b1 = blk(k + 1, n), b2 = blk(k + 2, n);
  const int64_t W = b.r1 - b.r0;
  const int64_t lda = w.lda, ldl = w.ldl;
  const int B = (int)w.B;
  const int64_t rest = n - b2.r0;   // rows > k + 1
  float* Arest = w.Aw + b2.r0 * lda + b.r0;
  SegStrides a3;
  a3.src = w.sAw; a3.dst = w.sAS2;
  RC(split_seg(s, B, Arest, lda, rest, W, w.AS2, 3 * GB, 3, 0b010, a3));
  RC(gemm(s, MATH_BF16, rest, W, 3 * W, 1.0f, A_n(w.AS2, DT_BF16, 3 * GB, TRI_NONE, w.sAS2),
          B_t(w.MT3[k & 1], DT_BF16, 3 * GB, TRI_NONE, w.sMT3), 0.0f,
          per_entry(out_f32(Arest, lda, w.sAw)), B, w.sp2, max_wgs));
  const int64_t k0 = 3 * GB * k;
  SegStrides l2;
  l2.src = w.sAw; l2.dst = w.sL; l2.dst2 = w.sL;
  RC(split_seg(s, B, w.Aw + b1.r0 * lda + b.r0, lda, n - b1.r0, W, w.LA + b1.r0 * ldl + k0, ldl,
               3, 0b010, l2, w.LB + b1.r0 * ldl + k0, ldl, 0b001));
  // column k + 1, rows > k + 1, by panel k
  if (gev_k1) HIPRC(hipStreamWaitEvent(s, gev_k1, 0), "fold_finalize_gram: stream wait failed");
  const int64_t W1 = b1.r1 - b1.r0;
  RC(gemm(s, MATH_BF16, rest, W1, 3 * GB, -1.0f,
          A_n(w.LA + b2.r0 * ldl + k0, DT_BF16, ldl, TRI_NONE, w.sL),
          B_t(w.LB + b1.r0 * ldl + k0, DT_BF16, ldl, TRI_NONE, w.sL), 1.0f,
          per_entry(out_f32(w.Aw + b2.r0 * lda + b1.r0, lda, w.sAw)), B, w.sp2, max_wgs));
  // block (k + 2, k + 1) is final: the next band's split copy, off the chain
  RC(split_band(s, w, n, k + 1));
  // column k + 2 by panels 0 .. k
  if (gev_k2) HIPRC(hipStreamWaitEvent(s, gev_k2, 0), "fold_finalize_gram: stream wait failed");
  const int64_t W2 = b2.r1 - b2.r0;
  return gemm(s, MATH_BF16, rest, W2, 3 * GB * (k + 1), -1.0f,
              A_n(w.LA + b2.r0 * ldl, DT_BF16, ldl, TRI_NONE, w.sL),
              B_t(w.LB + b2.r0 * ldl, DT_BF16, ldl, TRI_NONE, w.sL), 1.0f,
              per_entry(lower_part(out_f32(w.Aw + b2.r0 * lda + b2.r0, lda, w.sAw))), B, w.sp2, max_wgs);
}

// The inverse of the factor, Z = R^{-1}, and its bf16 copies, after the
// factorisation: the diagonal blocks are Z_jj = M_j / scale from the chain's
// M_j = U_jj^{-1} (U = L^T; the output R is scale U), and the block-doubling
// levels Z12 = -Z11 (R12 Z22) of the bf16 triangular inverse start at width
// GB instead of at its 64-column leaves.
int inverse_clear(hipStream_t s, const GramInverse& o, int64_t n, int B) {
  for (int e = 0; e < B; ++e) {
    RC(launch_zero_tri_blocks(s, o.Z + e * o.sz, 4, o.ldz, n, true));
    RC(launch_zero_tri_blocks(s, o.Zb + e * o.sb, 2, o.ldb, n, true));
    RC(launch_zero_tri_blocks(s, o.ZT + e * o.sb, 2, o.ldb, n, false));
  }
  return IFK_OK;
}

int inverse_from_blocks(hipStream_t s, GramWs& w, int64_t n, float scale, const void* out,
                        int odt, int64_t ldo, int64_t out_stride, const GramInverse& o) {
  const int B = (int)w.B;
  const int64_t nb = cdiv(n, GB);
  RC(inverse_clear(s, o, n, B));
  for (int64_t j = 0; j < nb; ++j) {
    const Blk b = blk(j, n);
    const int64_t W = b.r1 - b.r0, r = b.r0;
    const dim3 grid((unsigned)cdiv(W, 32), (unsigned)cdiv(W, 32), (unsigned)B);
    hipLaunchKernelGGL(diag_inverse_kernel, grid, dim3(256), 0, s, w.Mh + j * GB * GB, GB, W,
                       1.0f / scale, o.Z + r * o.ldz + r, o.ldz, o.Zb + r * o.ldb + r,
                       o.ZT + r * o.ldb + r, o.ldb, w.sMh, o.sz, o.sb);
    RC(check_launch("diag_inverse"));
  }
  const size_t esz = odt == DT_F32 ? 4 : 2;
  for (int e = 0; e < B; ++e)
    RC(trinv_levels_t(s, (const char*)out + (size_t)e * out_stride * esz, odt, ldo, n, GB,
                      o.Z + e * o.sz, o.ldz, o.ZT + e * o.sb, o.Zb + e * o.sb, o.ldb, w.Tinv,
                      w.sp2));
  return IFK_OK;
}

}  // namespace

size_t fold_finalize_gram_inv_ws(int64_t batch, int64_t p, int64_t n, int64_t r_in) {
  Arena a(nullptr, 0);
  GramWs w;
  plan_gram(a, batch, p, r_in, n, w, true);
  return a.used;
}

size_t fold_finalize_gram_ws(int64_t batch, int64_t p, int64_t n, int64_t r_in, bool split_r) {
  Arena a(nullptr, 0);
  GramWs w;
  plan_gram(a, batch, p, r_in, n, w, false, split_r);
  return a.used;
}

int fold_finalize_gram(hipStream_t s, int64_t batch, const void* const* X, int xdt, int64_t p,
                       int64_t n, int64_t ldx, const float* const* R_in, int64_t ldr,
                       int64_t r_in, float scale, float damping, void* out, int odt, int64_t ldo,
                       int64_t out_stride, int math, int* status, float* kappa_bound, void* ws,
                       size_t ws_bytes, float pivot_tol, const GramInverse* inv,
                       bool split_r) {
  bool ok = n >= 1 && p >= 0 && r_in >= 0 && r_in <= n && batch >= 1 && batch <= 65535 &&
            (p == 0 || (X && ldx >= n)) && (r_in == 0 || (R_in && ldr >= n)) && out &&
            ldo >= n && out_stride >= n * ldo && scale > 0.0f && damping >= 0.0f &&
            (xdt == DT_F32 || xdt == DT_BF16) && (odt == DT_F32 || odt == DT_BF16) && status;
  for (int64_t e = 0; ok && e < batch; ++e)
    ok = (p == 0 || X[e]) && (r_in == 0 || R_in[e]);
  if (ok && inv)
    ok = inv->Z && inv->Zb && inv->ZT && inv->ldz >= n && inv->ldb >= n &&
         (batch == 1 || (inv->sz >= n * inv->ldz && inv->sb >= n * inv->ldb));
  if (!ok) {
    set_error("fold_finalize_gram: invalid arguments");
    return IFK_ERR_INVALID;
  }
  if (math != MATH_BF16) {
    set_error("fold_finalize_gram: bf16 arithmetic only (fp32 arithmetic folds by "
              "ifk_fold_finalize_cqr / ifk_fold_finalize)");
    return IFK_ERR_INVALID;
  }
  const int64_t pe = r_in + p;
  if (!(damping > 0.0f) && pe < n) {
    set_error("fold_finalize_gram: fewer rows than columns and no damping (the factor is not "
              "square)");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  GramWs w;
  plan_gram(a, batch, p, r_in, n, w, inv != nullptr, split_r);
  const int64_t ke = w.kr + p;   // K extent of the Gram products
  if (a.overflow) {
    set_error("fold_finalize_gram: workspace too small");
    return IFK_ERR_WORKSPACE;
  }
  if (!(pivot_tol > 0.0f && pivot_tol < 1.0f)) {
    set_error("fold_finalize_gram: pivot tolerance outside (0, 1)");
    return IFK_ERR_INVALID;
  }
  w.tol = pivot_tol;
  const int B = (int)batch;
  const int64_t nb = cdiv(n, GB);
  LookAhead* la = nullptr;
  int rc = IFK_OK;
  if (nb > 2) {   // helper streams: the Gram columns, and the panel work beside the chain
    la = look_ahead(s, &rc);
    if (!la) return rc;
  }
  std::unique_lock<std::mutex> lock;
  if (la) {
    lock = std::unique_lock<std::mutex>(la->mu);
    RC(look_ahead_events(la, (size_t)nb));
  }
  hipStream_t s2 = la ? la->s2 : s, s3 = la ? la->s3 : s;
  const int wg2 = la ? REST_MAX_WGS : 0, wg3 = la ? GRAM_MAX_WGS : 0;
  const float c2 = damping / (scale * scale);
  const bool have_rows = pe > 0;
  for (int e = 0; e < B; ++e) RC(launch_fill_int(s, w.flag + e * FLAG_S, 0, 1));
  // P^T of each entry (bf16, K-padded with zeros): the running factor's rows
  // and the chunk's first column block on s, so that column 0's diagonal
  // block (all the chain's first step needs) can start; the chunk's other
  // column blocks go on s3 ahead of the rest of the Gram columns.
  const Blk b0 = blk(0, n);
  auto x_cols = [&](hipStream_t st, int64_t c0, int64_t c1) -> int {
    for (int e = 0; e < B; ++e) {
      const char* Xe = (const char*)X[e] + c0 * (xdt == DT_BF16 ? 2 : 4);
      for (bf16_t* base : {w.PT, w.PB}) {
        bf16_t* PT = base + e * w.sPT + c0 * w.ldk + w.kr;
        // a bf16 chunk moves as 32-bit pairs through a 64 x 64 tile
        if (xdt == DT_BF16)
          RC(launch_transpose_bf16(st, (const bf16_t*)Xe, ldx, p, c1 - c0, PT, w.ldk));
        else
          RC(transpose_to_bf16(st, Xe, xdt, ldx, p, c1 - c0, PT, w.ldk, false));
        if (w.PB == w.PT) break;
      }
    }
    return IFK_OK;
  };
  const bool two = w.PB != w.PT;
  for (int e = 0; e < B; ++e) {
    bf16_t* PT = w.PT + e * w.sPT;
    bf16_t* PB = w.PB + e * w.sPT;
    if (w.ldk > ke) {
      RC(launch_zero_bf16(s, PT + ke, w.ldk, n, w.ldk - ke));
      if (two) RC(launch_zero_bf16(s, PB + ke, w.ldk, n, w.ldk - ke));
    }
    if (r_in > 0)
      RC(transpose_to_bf16(s, R_in[e], DT_F32, ldr, r_in, n, PT, w.ldk, true,
                           two ? PB : nullptr));
  }
  if (p > 0) RC(x_cols(s, b0.r0, b0.r1));
  if (la) {
    HIPRC(hipEventRecord(la->ready[0], s), "fold_finalize_gram: event record failed");
    HIPRC(hipStreamWaitEvent(s3, la->ready[0], 0), "fold_finalize_gram: stream wait failed");
  }
  // Gram columns in order on s3, each with its event (they depend on P^T
  // only).  The chain's first step goes right behind column 0's diagonal
  // block: enqueued before the other columns, it does not wait for the host
  // to launch them.
  RC(gram_column0_diag(s3, w, n, c2, have_rows, wg3));
  if (la) {
    HIPRC(hipEventRecord(la->tready[0], s3), "fold_finalize_gram: event record failed");
    HIPRC(hipStreamWaitEvent(s, la->tready[0], 0), "fold_finalize_gram: stream wait failed");
  }
  RC(chain_factor(s, w, n, 0));
  if (p > 0 && n > b0.r1) RC(x_cols(s3, b0.r1, n));
  RC(gram_column0_rest(s3, w, n, have_rows, wg3));
  if (la) HIPRC(hipEventRecord(la->col[0], s3), "fold_finalize_gram: event record failed");
  // the columns before the lead (all of them without helper streams); the
  // rest are enqueued in the loop below, each behind its helper step
  const int64_t c_pre = la ? std::min<int64_t>(nb, GRAM_LEAD) : nb;
  for (int64_t c = 1; c < c_pre; ++c) {
    RC(gram_column(s3, w, n, c, c2, have_rows, wg3));
    if (la) HIPRC(hipEventRecord(la->col[c], s3), "fold_finalize_gram: event record failed");
  }
  // The chain on s; the helper s2 works one step behind it.  Events (each
  // recorded again only after the wait on its previous record is enqueued):
  //   tready[0]:     column 0's diagonal block done (s3)
  //   col[c]:        Gram column c done (s3)
  //   ready[k % 2]:  step k's band and diagonal update done (s -> s2)
  //   aready[k % 2]: helper step k done (s2 -> s, before step k + 1's band)
  for (int64_t k = 0; k < nb; ++k) {
    const int kp = (int)(k & 1);
    if (k > 0) RC(chain_factor(s, w, n, k));
    if (k + 1 >= nb) break;
    // the band of step k needs helper step k - 1 (column k's rows > k, and
    // column k + 1 updated by panels < k), which also frees MT3[k % 2]
    if (la && k >= 1 && k + 1 < nb)
      HIPRC(hipStreamWaitEvent(s, la->aready[kp ^ 1], 0), "fold_finalize_gram: stream wait failed");
    if (la && k == 0) {
      HIPRC(hipStreamWaitEvent(s, la->col[0], 0), "fold_finalize_gram: stream wait failed");
      HIPRC(hipStreamWaitEvent(s, la->col[1], 0), "fold_finalize_gram: stream wait failed");
    }
    RC(chain_band(s, w, n, k));
    if (k + 2 < nb) {
      if (la) {
        HIPRC(hipEventRecord(la->ready[kp], s), "fold_finalize_gram: event record failed");
        HIPRC(hipStreamWaitEvent(s2, la->ready[kp], 0), "fold_finalize_gram: stream wait failed");
      }
      RC(helper_step(s2, w, n, k, la ? la->col[k + 2] : nullptr,
                     (la && k == 0) ? la->col[1] : nullptr, wg2));
      if (la) HIPRC(hipEventRecord(la->aready[kp], s2), "fold_finalize_gram: event record failed");
      // Gram column k + GRAM_LEAD behind helper step k (every column >=
      // GRAM_LEAD comes here: k + 2 < nb holds for k = c - GRAM_LEAD)
      const int64_t c = k + GRAM_LEAD;
      if (la && c < nb) {
        HIPRC(hipStreamWaitEvent(s3, la->aready[kp], 0), "fold_finalize_gram: stream wait failed");
        RC(gram_column(s3, w, n, c, c2, have_rows, wg3));
        HIPRC(hipEventRecord(la->col[c], s3), "fold_finalize_gram: event record failed");
      }
    }
  }
  if (la) {
    HIPRC(hipEventRecord(la->done, s2), "fold_finalize_gram: event record failed");
    HIPRC(hipStreamWaitEvent(s, la->done, 0), "fold_finalize_gram: stream wait failed");
    HIPRC(hipEventRecord(la->fall[0], s3), "fold_finalize_gram: event record failed");
    HIPRC(hipStreamWaitEvent(s, la->fall[0], 0), "fold_finalize_gram: stream wait failed");
  }
  RC(launch_fill_int(s, status, 1, B));
  RC(cast_lower_t(s, B, w.Aw, w.lda, n, scale, out, odt, ldo, status, w.sAw, out_stride));
  if (inv) RC(inverse_from_blocks(s, w, n, scale, out, odt, ldo, out_stride, *inv));
  if (kappa_bound) {
    hipLaunchKernelGGL(kappa_bound_kernel, dim3((unsigned)B), dim3(256), 0, s, w.frob,
                       (int)w.sfrob, scale, damping, kappa_bound);
    RC(check_launch("kappa_bound"));
  }
  hipLaunchKernelGGL(status_merge_batch_kernel, dim3((unsigned)cdiv(B, 64)), dim3(64), 0, s,
                     status, w.flag, FLAG_S, B);
  return check_launch("status_merge");
}

// ---------------------------------------------------------------------------
// The streaming fold by the Gram route (bf16 arithmetic): R (n x n, rows
// [0, r_in) valid) becomes the factor of [R[0:r_in]; X] when that is square
// (r_in + p >= n).  The factor goes to the workspace first and is copied into
// R only where the status is 1, so a fold that fails the pivot test or meets
// non-finite input (status 2) leaves R as it was for the caller's panel fold.
// ---------------------------------------------------------------------------
namespace {

__global__ void cond_copy_kernel(const float* src, int64_t n, float* R, int64_t ldr,
                                 const int* status) {
  if (*status != 1) return;
  const int64_t total = n * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / n, j = e - i * n;
    R[i * ldr + j] = src[e];
  }
}

}  // namespace

size_t tsqr_fold_gram_ws(int64_t p, int64_t n, int64_t r_in) {
  return align_up((size_t)n * n * sizeof(float), 256) +
         fold_finalize_gram_ws(1, p, n, r_in, true);
}

int tsqr_fold_gram(hipStream_t s, const void* X, int xdt, int64_t p, int64_t n, int64_t ldx,
                   float* R, int64_t ldr, int64_t r_in, float pivot_tol, int* status, void* ws,
                   size_t ws_bytes) {
  if (n < 1 || p < 0 || r_in < 0 || r_in > n || r_in + p < n || !R || ldr < n || !status ||
      (p > 0 && (!X || ldx < n))) {
    set_error("tsqr_fold_gram: invalid arguments (the folded factor must be square: "
              "r_in + p >= n)");
    return IFK_ERR_INVALID;
  }
  const size_t head = align_up((size_t)n * n * sizeof(float), 256);
  if (!ws || ws_bytes < head) {
    set_error("tsqr_fold_gram: workspace too small");
    return IFK_ERR_WORKSPACE;
  }
  float* tmp = (float*)ws;
  const void* xs[1] = {X};
  const float* rs[1] = {R};
  RC(fold_finalize_gram(s, 1, xs, xdt, p, n, ldx, rs, ldr, r_in, 1.0f, 0.0f, tmp, DT_F32, n,
                        n * n, MATH_BF16, status, nullptr, (char*)ws + head, ws_bytes - head,
                        pivot_tol, nullptr, true));
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(n * n, 256), 4096);
  hipLaunchKernelGGL(cond_copy_kernel, dim3(blocks), dim3(256), 0, s, tmp, n, R, ldr, status);
  return check_launch("tsqr_fold_gram copy");
}

size_t tsqr_fold_gram_batched_ws(int64_t batch, int64_t p, int64_t n, int64_t r_in) {
  return align_up((size_t)batch * n * n * sizeof(float), 256) +
         fold_finalize_gram_ws(batch, p, n, r_in, true);
}

int tsqr_fold_gram_batched(hipStream_t s, int64_t batch, const void* const* X, int xdt,
                           int64_t p, int64_t n, int64_t ldx, float* const* R, int64_t ldr,
                           int64_t r_in, float pivot_tol, int* status, void* ws,
                           size_t ws_bytes) {
  bool ok = batch >= 1 && batch <= 65535 && n >= 1 && p >= 0 && r_in >= 0 && r_in <= n &&
            r_in + p >= n && R && X && ldr >= n && status && (p == 0 || ldx >= n);
  for (int64_t e = 0; ok && e < batch; ++e) ok = R[e] && (p == 0 || X[e]);
  if (!ok) {
    set_error("tsqr_fold_gram_batched: invalid arguments (the folded factors must be square: "
              "r_in + p >= n)");
    return IFK_ERR_INVALID;
  }
  const size_t head = align_up((size_t)batch * n * n * sizeof(float), 256);
  if (!ws || ws_bytes < head) {
    set_error("tsqr_fold_gram_batched: workspace too small");
    return IFK_ERR_WORKSPACE;
  }
  float* tmp = (float*)ws;
  RC(fold_finalize_gram(s, batch, X, xdt, p, n, ldx, (const float* const*)R, ldr, r_in, 1.0f,
                        0.0f, tmp, DT_F32, n, n * n, MATH_BF16, status, nullptr,
                        (char*)ws + head, ws_bytes - head, pivot_tol, nullptr, true));
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(n * n, 256), 4096);
  for (int64_t e = 0; e < batch; ++e) {
    hipLaunchKernelGGL(cond_copy_kernel, dim3(blocks), dim3(256), 0, s, tmp + e * n * n, n, R[e],
                       ldr, status + e);
    RC(check_launch("tsqr_fold_gram_batched copy"));
  }
  return IFK_OK;
}

}  // namespace ifk
