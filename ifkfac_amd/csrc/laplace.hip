// The Laplace consumer of the factors: their eigendecomposition and the
// posterior weight samples.
//
// Eigendecomposition of a factor's Gram matrix from the factor itself:
// R^T R = V diag(sigma^2) V^T, with V and sigma the right singular vectors
// and singular values of the n x n factor R, by one-sided block Jacobi on
// R's columns.  Working on R keeps the relative accuracy of kappa(R) rather
// than that of the formed Gram matrix's kappa(R)^2 (the reason the factor
// path exists), which is how the Laplace posterior's K-FAC eigenbasis is
// meant to come out of an IFKFAC factor (ifkfac/laplace.py:26-30).
//
// Layout.  S holds R's columns as rows (S[k][:] = R[:, k], n floats, rows
// padded with zeros to nb * JB), Vt the accumulated rotations the same way
// (Vt[k][:] = V[:, k], starting from I).  A sweep pairs every two blocks of
// JB columns once, in the round-robin ("circle") order: nb - 1 rounds, each
// one launch of nb / 2 workgroups, one per disjoint pair of blocks.  For its
// pair a workgroup forms the 2 JB x 2 JB Gram matrix G = P P^T of the pair's
// rows (accumulated in double), measures its largest relative off-diagonal
// |G_ij| / sqrt(G_ii G_jj), and, when that exceeds the tolerance,
// diagonalises G by cyclic Jacobi in LDS (double) and rotates the pair's
// rows of S and Vt by the eigenvector matrix.  The largest measure of a sweep
// decides convergence (sqrt(n) eps_fp32, LAPACK xGESVJ's test); the launches
// after it return at once.  Then sigma_k = ||S[k][:]||, sorted descending.
#include <algorithm>
#include <cmath>
#include <cstdint>

#include "gemm.h"
#include "kernels.h"
#include "linalg.h"

namespace ifk {

#define RC(x)                 \
  do {                        \
    int _rc = (x);            \
    if (_rc) return _rc;      \
  } while (0)

namespace {

constexpr int JB = 16;            // columns per block
constexpr int JP = 2 * JB;        // columns of a pair
constexpr int KC = 256;           // S columns staged per LDS chunk
constexpr int MAX_SWEEPS = 24;    // outer sweeps launched (the converged ones return at once)
constexpr int INNER_SWEEPS = 6;   // at most, for a pair's 2 JB x 2 JB Gram matrix

// block at position k of the circle in round r: position nb - 1 is fixed
__device__ inline int circle_block(int k, int r, int nb) {
  return k == nb - 1 ? nb - 1 : (k + r) % (nb - 1);
}

// float >= 0 as an order-preserving uint (atomicMax on the bits)
__device__ inline unsigned fbits(float f) { return __float_as_uint(f); }

__global__ __launch_bounds__(256) void jacobi_round_kernel(float* S, float* Vt, int64_t n, int nb,
                                                           int round, unsigned* off_sweep,
                                                           const int* done, float tol) {
  if (*done) return;
  __shared__ float Ps[JP][KC + 1];
  __shared__ double G[JP][JP + 1];
  __shared__ double Q[JP][JP + 1];
  __shared__ float Qf[JP][JP];
  __shared__ double cs[JP / 2][2];
  __shared__ int pidx[JP / 2][2];
  __shared__ float red[256];
  __shared__ int rot_flag;

  const int t = threadIdx.x;
  const int w = blockIdx.x;
  const int bi = circle_block(w, round, nb), bj = circle_block(nb - 1 - w, round, nb);
  // row of S for the pair's local column l
  auto prow = [&](int l) -> int64_t {
    return (int64_t)(l < JB ? bi * JB + l : bj * JB + (l - JB));
  };

  // ---- G = P P^T in double: thread t owns row gi, columns gj0 .. gj0 + 3
  const int gi = t >> 3, gj0 = (t & 7) * 4;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  for (int64_t c0 = 0; c0 < n; c0 += KC) {
    const int kc = (int)std::min<int64_t>(KC, n - c0);
    __syncthreads();
    for (int e = t; e < JP * KC; e += 256) {
      const int l = e / KC, cc = e - l * KC;
      Ps[l][cc] = cc < kc ? S[prow(l) * n + c0 + cc] : 0.0f;
    }
    __syncthreads();
    for (int cc = 0; cc < kc; ++cc) {
      const double a = (double)Ps[gi][cc];
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] = fma(a, (double)Ps[gj0 + u][cc], acc[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) G[gi][gj0 + u] = acc[u];
  __syncthreads();

  // ---- largest relative off-diagonal of the pair
  float m = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int j = gj0 + u;
    if (j != gi) {
      const double d = G[gi][gi] * G[j][j];
      const double o = fabs(G[gi][j]);
      if (o > 0.0) m = fmaxf(m, d > 0.0 ? (float)(o / sqrt(d)) : 1.0f);
    }
  }
  red[t] = m;
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if (t < h) red[t] = fmaxf(red[t], red[t + h]);
    __syncthreads();
  }
  const float pair_off = red[0];
  if (t == 0) {
    atomicMax(off_sweep, fbits(pair_off));
    rot_flag = pair_off > tol ? 1 : 0;
  }
  __syncthreads();
  if (!rot_flag) return;

  // ---- cyclic Jacobi on G (double), eigenvectors accumulated in Q
  for (int e = t; e < JP * JP; e += 256) {
    const int i = e / JP, j = e - i * JP;
    Q[i][j] = i == j ? 1.0 : 0.0;
  }
  __syncthreads();
  for (int sweep = 0; sweep < INNER_SWEEPS; ++sweep) {
    for (int step = 0; step < JP - 1; ++step) {
      // the JP / 2 disjoint pairs of this step: positions t and JP - 1 - t
      if (t < JP / 2) {
        const int pa = circle_block(t, step, JP), pb = circle_block(JP - 1 - t, step, JP);
        const double app = G[pa][pa], aqq = G[pb][pb], apq = G[pa][pb];
        double c = 1.0, s = 0.0;
        if (fabs(apq) > 1e-300 && fabs(apq) > 1e-17 * sqrt(fabs(app * aqq))) {
          // Golub & Van Loan's symmetric 2 x 2 Schur rotation: (J^T G J)_pq = 0
          const double tau = (aqq - app) / (2.0 * apq);
          const double tt = (tau >= 0.0 ? 1.0 : -1.0) / (fabs(tau) + sqrt(1.0 + tau * tau));
          c = 1.0 / sqrt(1.0 + tt * tt);
          s = tt * c;
        }
        cs[t][0] = c;
        cs[t][1] = s;
        pidx[t][0] = pa;
        pidx[t][1] = pb;
      }
      __syncthreads();
      // rows of G (G <- J^T G) and columns of Q (Q <- Q J)
      for (int e = t; e < (JP / 2) * JP; e += 256) {
        const int r = e / JP, k = e - r * JP;
        const int pa = pidx[r][0], pb = pidx[r][1];
        const double c = cs[r][0], s = cs[r][1];
        const double gp = G[pa][k], gq = G[pb][k];
        G[pa][k] = c * gp - s * gq;
        G[pb][k] = s * gp + c * gq;
        const double qp = Q[k][pa], qq = Q[k][pb];
        Q[k][pa] = c * qp - s * qq;
        Q[k][pb] = s * qp + c * qq;
      }
      __syncthreads();
      // columns of G (G <- G J)
      for (int e = t; e < (JP / 2) * JP; e += 256) {
        const int r = e / JP, k = e - r * JP;
        const int pa = pidx[r][0], pb = pidx[r][1];
        const double c = cs[r][0], s = cs[r][1];
        const double gp = G[k][pa], gq = G[k][pb];
        G[k][pa] = c * gp - s * gq;
        G[k][pb] = s * gp + c * gq;
      }
      __syncthreads();
    }
    // converged pair: every relative off-diagonal below a tenth of the tolerance
    float mm = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = gj0 + u;
      if (j != gi) {
        const double d = G[gi][gi] * G[j][j];
        const double o = fabs(G[gi][j]);
        if (o > 0.0) mm = fmaxf(mm, d > 0.0 ? (float)(o / sqrt(d)) : 1.0f);
      }
    }
    __syncthreads();
    red[t] = mm;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
      if (t < h) red[t] = fmaxf(red[t], red[t + h]);
      __syncthreads();
    }
    const bool conv = red[0] <= 0.1f * tol;
    __syncthreads();
    if (conv) break;
  }
  for (int e = t; e < JP * JP; e += 256) {
    const int i = e / JP, j = e - i * JP;
    Qf[i][j] = (float)Q[i][j];
  }
  __syncthreads();

  // ---- rotate the pair's rows of S and Vt: row' r = sum_k Q[k][r] row k
  for (int pass = 0; pass < 2; ++pass) {
    float* M = pass == 0 ? S : Vt;
    for (int64_t c0 = 0; c0 < n; c0 += KC) {
      const int kc = (int)std::min<int64_t>(KC, n - c0);
      __syncthreads();
      for (int e = t; e < JP * KC; e += 256) {
        const int l = e / KC, cc = e - l * KC;
        Ps[l][cc] = cc < kc ? M[prow(l) * n + c0 + cc] : 0.0f;
      }
      __syncthreads();
      const int cc = t;   // KC == blockDim
      if (cc < kc) {
        float in[JP];
#pragma unroll
        for (int k = 0; k < JP; ++k) in[k] = Ps[k][cc];
#pragma unroll 4
        for (int r = 0; r < JP; ++r) {
          float o = 0.0f;
#pragma unroll
          for (int k = 0; k < JP; ++k) o = fmaf(Qf[k][r], in[k], o);
          M[prow(r) * n + c0 + cc] = o;
        }
      }
    }
  }
}

// after sweep `sweep`: converged when its largest measure is <= tol
__global__ void sweep_end_kernel(const unsigned* off, int sweep, float tol, int* done,
                                 int* sweeps) {
  if (threadIdx.x != 0 || *done) return;
  if (__uint_as_float(off[sweep]) <= tol) {
    *done = 1;
    *sweeps = sweep + 1;
  } else {
    *sweeps = -(sweep + 1);   // not (yet) converged
  }
}

// sig2[k] = ||S[k][:]||^2 (double), one workgroup per row
__global__ __launch_bounds__(256) void row_norm2_kernel(const float* S, int64_t n, double* sig2) {
  __shared__ double red[256];
  const int64_t k = blockIdx.x;
  double a = 0.0;
  for (int64_t c = threadIdx.x; c < n; c += 256) {
    const double v = S[k * n + c];
    a = fma(v, v, a);
  }
  red[threadIdx.x] = a;
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if ((int)threadIdx.x < h) red[threadIdx.x] += red[threadIdx.x + h];
    __syncthreads();
  }
  if (threadIdx.x == 0) sig2[k] = red[0];
}

// rank of each value in descending order (ties by index)
__global__ void rank_desc_kernel(const double* v, int64_t n, int* rank) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const double x = v[i];
  int r = 0;
  for (int64_t j = 0; j < n; ++j) {
    const double y = v[j];
    r += (y > x || (y == x && j < i)) ? 1 : 0;
  }
  rank[i] = r;
}

// V[:, rank[k]] = Vt[k][:], eig[rank[k]] = sig2[k]
__global__ __launch_bounds__(256) void scatter_evd_kernel(const float* Vt, int64_t n,
                                                          const int* rank, const double* sig2,
                                                          float* V, int64_t ldv, float* eig) {
  __shared__ float tile[32][33];
  const int64_t k0 = (int64_t)blockIdx.y * 32, r0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int a = ty; a < 32; a += 8) {
    const int64_t k = k0 + a, r = r0 + tx;
    tile[a][tx] = (k < n && r < n) ? Vt[k * n + r] : 0.0f;
  }
  __syncthreads();
  for (int a = ty; a < 32; a += 8) {
    const int64_t r = r0 + a, k = k0 + tx;
    if (k < n && r < n) V[r * ldv + rank[k]] = tile[tx][a];
  }
  if (blockIdx.x == 0 && threadIdx.x < 32) {
    const int64_t k = k0 + threadIdx.x;
    if (k < n) eig[rank[k]] = (float)sig2[k];
  }
}

struct EvdWs {
  int nb;
  float* S;
  float* Vt;
  unsigned* off;
  int* done;
  double* sig2;
  int* rank;
};

void plan_evd(Arena& a, int64_t n, EvdWs& w) {
  int64_t nb = cdiv(n, JB);
  if (nb < 2) nb = 2;
  if (nb & 1) ++nb;
  w.nb = (int)nb;
  const int64_t m = nb * JB;
  w.S = a.take<float>((size_t)m * n);
  w.Vt = a.take<float>((size_t)m * n);
  w.off = a.take<unsigned>(MAX_SWEEPS);
  w.done = a.take<int>(1);
  w.sig2 = a.take<double>((size_t)n);
  w.rank = a.take<int>((size_t)n);
}

}  // namespace

size_t factor_evd_ws(int64_t n) {
  Arena a(nullptr, 0);
  EvdWs w;
  plan_evd(a, n, w);
  return a.used;
}

int factor_evd(hipStream_t s, const void* R, int rdt, int64_t ldr, int64_t n, float* V,
               int64_t ldv, float* eig, int* sweeps, void* ws, size_t ws_bytes) {
  if (n < 1 || ldr < n || ldv < n || !R || !V || !eig || !sweeps || n > (int64_t)1 << 20) {
    set_error("factor_evd: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  EvdWs w;
  plan_evd(a, n, w);
  if (a.overflow) {
    set_error("factor_evd: workspace too small");
    return IFK_ERR_WORKSPACE;
  }
  const int64_t m = (int64_t)w.nb * JB;
  // S = R^T (upper triangle of R only), padding rows zero; Vt = I
  RC(launch_zero(s, w.S, n, m, n));
  RC(launch_transpose_to_f32(s, R, rdt, ldr, n, n, w.S, n, true));
  RC(launch_zero(s, w.Vt, n, m, n));
  RC(launch_set_diag(s, w.Vt, n, n, 1.0f));
  RC(launch_fill_int(s, (int*)w.off, 0, MAX_SWEEPS));
  RC(launch_fill_int(s, w.done, 0, 1));
  RC(launch_fill_int(s, sweeps, 0, 1));
  const float tol = (float)(std::sqrt((double)n) * 1.1920929e-7);
  for (int sw = 0; sw < MAX_SWEEPS; ++sw) {
    for (int r = 0; r < w.nb - 1; ++r) {
      hipLaunchKernelGGL(jacobi_round_kernel, dim3(w.nb / 2), dim3(256), 0, s, w.S, w.Vt, n, w.nb,
                         r, w.off + sw, w.done, tol);
      RC(check_launch("factor_evd round"));
    }
    hipLaunchKernelGGL(sweep_end_kernel, dim3(1), dim3(64), 0, s, w.off, sw, tol, w.done, sweeps);
    RC(check_launch("factor_evd sweep end"));
  }
  hipLaunchKernelGGL(row_norm2_kernel, dim3((unsigned)n), dim3(256), 0, s, w.S, n, w.sig2);
  RC(check_launch("factor_evd norms"));
  hipLaunchKernelGGL(rank_desc_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, s, w.sig2, n,
                     w.rank);
  RC(check_launch("factor_evd rank"));
  const dim3 grid((unsigned)cdiv(n, 32), (unsigned)cdiv(n, 32));
  hipLaunchKernelGGL(scatter_evd_kernel, grid, dim3(256), 0, s, w.Vt, n, w.rank, w.sig2, V, ldv,
                     eig);
  return check_launch("factor_evd scatter");
}

// ----------------------------------------------------------------------------
// Laplace posterior sampling (ifkfac/laplace.py:84-101, :112-158)
// ----------------------------------------------------------------------------
namespace {

// out[i] = 1 / sqrt(sqrt_n * d[i] + sqrt_lam)  (laplace.py:95-96)
__global__ void laplace_scales_kernel(const float* d, int64_t n, float sqrt_n, float sqrt_lam,
                                      float* out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = 1.0f / sqrtf(sqrt_n * d[i] + sqrt_lam);
}

// Y[i][j] = (X[i][j] * sl[i]) * sr[j]  (laplace.py:146-147, the same order)
__global__ void scale_rows_cols_kernel(const float* X, int64_t ldx, const float* sl,
                                       const float* sr, int64_t rows, int64_t cols, float* Y,
                                       int64_t ldy) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / cols, j = e - i * cols;
    Y[i * ldy + j] = (X[i * ldx + j] * sl[i]) * sr[j];
  }
}

size_t split_floats_for(int64_t m, int64_t n) {
  size_t f = (size_t)64 * 64 * std::max(m, n);
  const size_t cap = (size_t)16 << 20;
  return std::min(f, cap);
}

}  // namespace

int laplace_scales(hipStream_t s, const float* d, int64_t n, float sqrt_n, float sqrt_lam,
                   float* out) {
  if (n < 1 || !d || !out) {
    set_error("laplace_scales: invalid arguments");
    return IFK_ERR_INVALID;
  }
  hipLaunchKernelGGL(laplace_scales_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, s, d, n,
                     sqrt_n, sqrt_lam, out);
  return check_launch("laplace_scales");
}

size_t laplace_sample_ws(int64_t n_out, int64_t n_in) {
  Arena a(nullptr, 0);
  a.take<float>((size_t)n_out * n_in * 2);
  a.take<float>(split_floats_for(n_out, n_in));
  return a.used;
}

int laplace_sample(hipStream_t s, const float* W_map, int64_t ldm, float* W, int64_t ldw,
                   int64_t n_out, int64_t n_in, const float* U_G, int64_t ldug, const float* s_G,
                   const float* U_A, int64_t ldua, const float* s_A, const float* Xi,
                   int64_t ldxi, void* ws, size_t ws_bytes) {
  if (n_out < 1 || n_in < 1 || ldm < n_in || ldw < n_in || ldug < n_out || ldua < n_in ||
      ldxi < n_in || !W_map || !W || !U_G || !s_G || !U_A || !s_A || !Xi) {
    set_error("laplace_sample: invalid arguments");
    return IFK_ERR_INVALID;
  }
  Arena a(ws, ws_bytes);
  float* Xs = a.take<float>((size_t)n_out * n_in);
  float* T = a.take<float>((size_t)n_out * n_in);
  SplitScratch sp;
  sp.floats = split_floats_for(n_out, n_in);
  sp.p = a.take<float>(sp.floats);
  if (a.overflow) {
    set_error("laplace_sample: workspace too small");
    return IFK_ERR_WORKSPACE;
  }
  const int64_t blocks = std::min<int64_t>(cdiv(n_out * n_in, 256), 65536);
  hipLaunchKernelGGL(scale_rows_cols_kernel, dim3((unsigned)blocks), dim3(256), 0, s, Xi, ldxi,
                     s_G, s_A, n_out, n_in, Xs, n_in);
  RC(check_launch("laplace_sample scale"));
  // W = W_map + (U_G Xs) U_A^T  (laplace.py:150-154), fp32 arithmetic
  RC(gemm(s, MATH_F32, n_out, n_in, n_out, 1.0f, A_n(U_G, DT_F32, ldug), B_n(Xs, DT_F32, n_in),
          0.0f, out_f32(T, n_in), 1, sp));
  if (W != W_map) RC(launch_copy_to_f32(s, W_map, DT_F32, ldm, n_out, n_in, 1.0f, W, ldw));
  return gemm(s, MATH_F32, n_out, n_in, n_in, 1.0f, A_n(T, DT_F32, n_in),
              B_t(U_A, DT_F32, ldua), 1.0f, out_f32(W, ldw), 1, sp);
}

}  // namespace ifk
