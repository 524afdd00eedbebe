// HBM-bound elementwise kernels: operand staging, masking, casts and the fused
// momentum / weight update.  Grid-stride loops over 256-thread blocks.
#include "kernels.h"

namespace ifk {

static inline unsigned grid_for(int64_t n) {
  int64_t g = cdiv(n, 256);
  if (g > 8192) g = 8192;
  if (g < 1) g = 1;
  return (unsigned)g;
}

template <int DT>
__global__ void copy_to_f32_kernel(const void* src, int64_t lds, int64_t rows, int64_t cols,
                                   float scale, float* dst, int64_t ldd) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / cols, c = e % cols;
    dst[r * ldd + c] =
        scale * Elem<DT>::load((const typename Elem<DT>::T*)src + r * lds + c);
  }
}

int launch_copy_to_f32(hipStream_t s, const void* src, int sdt, int64_t lds, int64_t rows,
                       int64_t cols, float scale, float* dst, int64_t ldd) {
  if (rows * cols == 0) return IFK_OK;
  if (sdt == DT_F32)
    hipLaunchKernelGGL(copy_to_f32_kernel<DT_F32>, dim3(grid_for(rows * cols)), dim3(256), 0, s,
                       src, lds, rows, cols, scale, dst, ldd);
  else
    hipLaunchKernelGGL(copy_to_f32_kernel<DT_BF16>, dim3(grid_for(rows * cols)), dim3(256), 0, s,
                       src, lds, rows, cols, scale, dst, ldd);
  return check_launch("copy_to_f32");
}

__global__ void copy_upper_kernel(const float* src, int64_t lds, int64_t n, float scale,
                                  float* dst, int64_t ldd) {
  const int64_t total = n * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / n, c = e % n;
    dst[r * ldd + c] = (c >= r) ? scale * src[r * lds + c] : 0.0f;
  }
}

int launch_copy_upper(hipStream_t s, const float* src, int64_t lds, int64_t n, float scale,
                      float* dst, int64_t ldd) {
  if (n == 0) return IFK_OK;
  hipLaunchKernelGGL(copy_upper_kernel, dim3(grid_for(n * n)), dim3(256), 0, s, src, lds, n, scale,
                     dst, ldd);
  return check_launch("copy_upper");
}

__global__ void set_diag_kernel(float* dst, int64_t ldd, int64_t n, float value) {
  const int64_t total = n * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / n, c = e % n;
    dst[r * ldd + c] = (r == c) ? value : 0.0f;
  }
}

int launch_set_diag(hipStream_t s, float* dst, int64_t ldd, int64_t n, float value) {
  if (n == 0) return IFK_OK;
  hipLaunchKernelGGL(set_diag_kernel, dim3(grid_for(n * n)), dim3(256), 0, s, dst, ldd, n, value);
  return check_launch("set_diag");
}

__global__ void zero_block_kernel(float* dst, int64_t ldd, int64_t rows, int64_t cols) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / cols, c = e % cols;
    dst[r * ldd + c] = 0.0f;
  }
}

int launch_zero_rows(hipStream_t s, float* dst, int64_t ldd, int64_t r0, int64_t r1,
                     int64_t cols) {
  if (r1 <= r0 || cols == 0) return IFK_OK;
  hipLaunchKernelGGL(zero_block_kernel, dim3(grid_for((r1 - r0) * cols)), dim3(256), 0, s,
                     dst + r0 * ldd, ldd, r1 - r0, cols);
  return check_launch("zero_rows");
}

int launch_zero(hipStream_t s, float* dst, int64_t ldd, int64_t rows, int64_t cols) {
  if (rows * cols == 0) return IFK_OK;
  hipLaunchKernelGGL(zero_block_kernel, dim3(grid_for(rows * cols)), dim3(256), 0, s, dst, ldd,
                     rows, cols);
  return check_launch("zero");
}

__global__ void zero_block_bf16_kernel(bf16_t* dst, int64_t ldd, int64_t rows, int64_t cols) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / cols, c = e % cols;
    dst[r * ldd + c] = 0;
  }
}

int launch_zero_bf16(hipStream_t s, bf16_t* dst, int64_t ldd, int64_t rows, int64_t cols) {
  if (rows * cols == 0) return IFK_OK;
  hipLaunchKernelGGL(zero_block_bf16_kernel, dim3(grid_for(rows * cols)), dim3(256), 0, s, dst,
                     ldd, rows, cols);
  return check_launch("zero_bf16");
}

// Zero the 64 x 64 blocks of an n x n matrix (element size es bytes, row
// stride ldb bytes) strictly below (lower) or above the block diagonal, one
// row per workgroup, 16-byte stores where the row allows.  The blocked
// triangular inverses write every block on and above (below, for the
// transposed copy) the diagonal, so only these need clearing.
__global__ void zero_tri_blocks_kernel(char* dst, int es, int64_t ldb, int64_t n, int lower,
                                       int vec) {
  for (int64_t r = blockIdx.x; r < n; r += gridDim.x) {
    const int64_t kb = (r / 64) * 64;
    const int64_t c0 = lower ? 0 : kb + 64, c1 = lower ? kb : n;
    if (c1 <= c0) continue;
    char* row = dst + r * ldb;
    const int64_t b0 = c0 * es, b1 = c1 * es;
    const int64_t v1 = vec ? b0 + (b1 - b0) / 16 * 16 : b0;
    for (int64_t b = b0 + (int64_t)threadIdx.x * 16; b < v1; b += (int64_t)blockDim.x * 16)
      *(uint4*)(row + b) = make_uint4(0, 0, 0, 0);
    for (int64_t b = v1 + (int64_t)threadIdx.x * es; b < b1; b += (int64_t)blockDim.x * es) {
      if (es == 4) *(uint32_t*)(row + b) = 0u;
      else *(uint16_t*)(row + b) = (uint16_t)0;
    }
  }
}

int launch_zero_tri_blocks(hipStream_t s, void* dst, int es, int64_t ld, int64_t n, bool lower) {
  if (n <= 64) return IFK_OK;
  if (es != 2 && es != 4) {
    set_error("zero_tri_blocks: element size");
    return IFK_ERR_INVALID;
  }
  // every block edge is a multiple of 64 elements, so 16-byte stores need
  // only an aligned base and row stride
  const int vec = ((uintptr_t)dst % 16 == 0) && ((ld * es) % 16 == 0);
  hipLaunchKernelGGL(zero_tri_blocks_kernel, dim3((unsigned)std::min<int64_t>(n, 4096)), dim3(256),
                     0, s, (char*)dst, es, ld * es, n, lower ? 1 : 0, vec);
  return check_launch("zero_tri_blocks");
}

// R[i][j] -= WT[j][i] over a rows x cols block, through a 32 x 32 LDS tile so
// both the read of WT and the update of R are coalesced.
__global__ void sub_transposed_kernel(float* R, int64_t ldr, const float* WT, int64_t ldw,
                                      int64_t rows, int64_t cols) {
  __shared__ float tile[32][33];
  const int64_t i0 = (int64_t)blockIdx.y * 32, j0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 256 threads: 32 x 8
  for (int k = ty; k < 32; k += 8) {
    const int64_t j = j0 + k, i = i0 + tx;
    tile[k][tx] = (j < cols && i < rows) ? WT[j * ldw + i] : 0.0f;
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t i = i0 + k, j = j0 + tx;
    if (i < rows && j < cols) R[i * ldr + j] -= tile[tx][k];
  }
}

int launch_sub_transposed(hipStream_t s, float* R, int64_t ldr, const float* WT, int64_t ldw,
                          int64_t rows, int64_t cols) {
  if (rows * cols == 0) return IFK_OK;
  if (cdiv(rows, 32) > 65535) {
    set_error("sub_transposed: too many rows");
    return IFK_ERR_INVALID;
  }
  hipLaunchKernelGGL(sub_transposed_kernel, dim3((unsigned)cdiv(cols, 32), (unsigned)cdiv(rows, 32)),
                     dim3(256), 0, s, R, ldr, WT, ldw, rows, cols);
  return check_launch("sub_transposed");
}

__global__ void sub_inplace_kernel(float* dst, int64_t ldd, const float* src, int64_t lds,
                                   int64_t rows, int64_t cols) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / cols, c = e % cols;
    dst[r * ldd + c] -= src[r * lds + c];
  }
}

int launch_sub_inplace(hipStream_t s, float* dst, int64_t ldd, const float* src, int64_t lds,
                       int64_t rows, int64_t cols) {
  if (rows * cols == 0) return IFK_OK;
  hipLaunchKernelGGL(sub_inplace_kernel, dim3(grid_for(rows * cols)), dim3(256), 0, s, dst, ldd,
                     src, lds, rows, cols);
  return check_launch("sub_inplace");
}

// One block per row (row-stride loop): read the diagonal, flip the row when
// it is negative.  Matches _positive_diagonal_R: sign 0 counts as +1.
__global__ void sign_normalize_kernel(float* R, int64_t ldr, int64_t r, int64_t n) {
  for (int64_t row = blockIdx.x; row < r; row += gridDim.x) {
    const float d = R[row * ldr + row];
    if (d < 0.0f) {
      for (int64_t c = threadIdx.x; c < n; c += blockDim.x) R[row * ldr + c] = -R[row * ldr + c];
    }
  }
}

int launch_sign_normalize(hipStream_t s, float* R, int64_t ldr, int64_t r, int64_t n) {
  if (r == 0) return IFK_OK;
  unsigned g = (unsigned)(r < 8192 ? r : 8192);
  hipLaunchKernelGGL(sign_normalize_kernel, dim3(g), dim3(256), 0, s, R, ldr, r, n);
  return check_launch("sign_normalize");
}

template <int ODT>
__global__ void cast_upper_kernel(const float* R, int64_t ldr, int64_t n, void* out, int64_t ldo,
                                  int* finite, float scale) {
  const int64_t total = n * n;
  bool ok = true;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / n, c = e % n;
    const float v = (c >= r) ? scale * R[r * ldr + c] : 0.0f;
    ok = ok && isfinite(v);
    if constexpr (ODT == DT_F32) ((float*)out)[r * ldo + c] = v;
    else ((bf16_t*)out)[r * ldo + c] = f32_to_bf16(v);
  }
  if (finite && !ok) atomicAnd(finite, 0);
}

int launch_cast_upper(hipStream_t s, const float* R, int64_t ldr, int64_t n, void* out, int odt,
                      int64_t ldo, int* finite, float scale) {
  if (n == 0) return IFK_OK;
  if (odt == DT_F32)
    hipLaunchKernelGGL(cast_upper_kernel<DT_F32>, dim3(grid_for(n * n)), dim3(256), 0, s, R, ldr, n,
                       out, ldo, finite, scale);
  else
    hipLaunchKernelGGL(cast_upper_kernel<DT_BF16>, dim3(grid_for(n * n)), dim3(256), 0, s, R, ldr,
                       n, out, ldo, finite, scale);
  return check_launch("cast_upper");
}

template <int ODT>
__global__ void cast_kernel(const float* src, int64_t lds, int64_t rows, int64_t cols, void* out,
                            int64_t ldo) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / cols, c = e % cols;
    const float v = src[r * lds + c];
    if constexpr (ODT == DT_F32) ((float*)out)[r * ldo + c] = v;
    else ((bf16_t*)out)[r * ldo + c] = f32_to_bf16(v);
  }
}

int launch_cast(hipStream_t s, const float* src, int64_t lds, int64_t rows, int64_t cols, void* out,
                int odt, int64_t ldo) {
  if (rows * cols == 0) return IFK_OK;
  if (odt == DT_F32)
    hipLaunchKernelGGL(cast_kernel<DT_F32>, dim3(grid_for(rows * cols)), dim3(256), 0, s, src, lds,
                       rows, cols, out, ldo);
  else
    hipLaunchKernelGGL(cast_kernel<DT_BF16>, dim3(grid_for(rows * cols)), dim3(256), 0, s, src, lds,
                       rows, cols, out, ldo);
  return check_launch("cast");
}

__global__ void fill_int_kernel(int* p, int value, int count) {
  for (int i = threadIdx.x; i < count; i += blockDim.x) p[i] = value;
}

int launch_fill_int(hipStream_t s, int* p, int value, int count) {
  if (count <= 0) return IFK_OK;
  hipLaunchKernelGGL(fill_int_kernel, dim3(1), dim3(64), 0, s, p, value, count);
  return check_launch("fill_int");
}

// dst[i] = src[i] for status words, dst in pinned host memory (its device
// address): one store per word at system scope, so the value is in host
// memory once the kernel has completed.
__global__ void status_to_host_kernel(const int* __restrict__ src, int* dst, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x)
    __hip_atomic_store(dst + i, src[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

int launch_status_to_host(hipStream_t s, const int* src, int* dst_dev, int n) {
  if (n <= 0) return IFK_OK;
  hipLaunchKernelGGL(status_to_host_kernel, dim3(1), dim3(64), 0, s, src, dst_dev, n);
  return check_launch("status_to_host");
}

// buf <- (buf_init ? nat : momentum * buf + nat)   [ifkfac.py:404-406]
// W   <- W * (1 - lr * wd) - lr * buf               [ifkfac.py:411-413]
// momentum == 0 uses nat directly and leaves buf untouched (buf may be null).
// 16 bytes per lane per access: float4 body, scalar tail.
__global__ void momentum_update_kernel(const float* __restrict__ nat, float* __restrict__ buf,
                                       float* __restrict__ W, int64_t numel, float lr,
                                       float momentum, float wd_scale, int buf_init, int use_buf,
                                       int vec) {
  const int64_t n4 = vec ? numel / 4 : 0;
  const float4* nat4 = (const float4*)nat;
  float4* buf4 = (float4*)buf;
  float4* W4 = (float4*)W;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * blockDim.x) {
    float4 g = nat4[i];
    float4 d = g;
    if (use_buf) {
      if (buf_init) {
        // zeros_like(nat).mul_(momentum).add_(nat): keeps torch's +0 for -0 inputs
        const float z = 0.0f * momentum;
        d.x = z + g.x; d.y = z + g.y; d.z = z + g.z; d.w = z + g.w;
      } else {
        const float4 b = buf4[i];
        d.x = momentum * b.x + g.x;
        d.y = momentum * b.y + g.y;
        d.z = momentum * b.z + g.z;
        d.w = momentum * b.w + g.w;
      }
      buf4[i] = d;
    }
    float4 w = W4[i];
    w.x = w.x * wd_scale - lr * d.x;
    w.y = w.y * wd_scale - lr * d.y;
    w.z = w.z * wd_scale - lr * d.z;
    w.w = w.w * wd_scale - lr * d.w;
    W4[i] = w;
  }
  for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel;
       i += (int64_t)gridDim.x * blockDim.x) {
    float d = nat[i];
    if (use_buf) {
      d = (buf_init ? 0.0f * momentum : momentum * buf[i]) + d;
      buf[i] = d;
    }
    W[i] = W[i] * wd_scale - lr * d;
  }
}

int launch_momentum_update(hipStream_t s, const float* nat, float* buf, float* W, int64_t numel,
                           float lr, float momentum, float weight_decay, int buf_init) {
  if (numel == 0) return IFK_OK;
  const int use_buf = momentum > 0.0f ? 1 : 0;
  if (use_buf && !buf) {
    set_error("momentum_update: momentum > 0 needs a buffer");
    return IFK_ERR_INVALID;
  }
  const int vec = (((uintptr_t)nat | (uintptr_t)W | (uintptr_t)(use_buf ? buf : W)) % 16 == 0);
  const float wd_scale = weight_decay > 0.0f ? 1.0f - lr * weight_decay : 1.0f;
  unsigned g = grid_for(cdiv(numel, 4));
  if (g > 2048) g = 2048;
  hipLaunchKernelGGL(momentum_update_kernel, dim3(g), dim3(256), 0, s, nat, buf, W, numel, lr,
                     momentum, wd_scale, buf_init, use_buf, vec);
  return check_launch("momentum_update");
}

template <int ODT>
__global__ void scale_copy_vec_kernel(const float* x, int64_t n, float alpha, void* out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float v = alpha * x[i];
    if constexpr (ODT == DT_F32) ((float*)out)[i] = v;
    else ((bf16_t*)out)[i] = f32_to_bf16(v);
  }
}

int launch_scale_copy_vec(hipStream_t s, const float* x, int64_t n, float alpha, void* out,
                          int odt) {
  if (n == 0) return IFK_OK;
  if (odt == DT_F32)
    hipLaunchKernelGGL(scale_copy_vec_kernel<DT_F32>, dim3(grid_for(n)), dim3(256), 0, s, x, n,
                       alpha, out);
  else
    hipLaunchKernelGGL(scale_copy_vec_kernel<DT_BF16>, dim3(grid_for(n)), dim3(256), 0, s, x, n,
                       alpha, out);
  return check_launch("scale_copy_vec");
}

// dst (cols x rows, fp32) = src^T through a 32 x 32 LDS tile: the read of
// src and the write of dst are both coalesced.
template <int DT>
__global__ void transpose_to_f32_kernel(const void* src, int64_t lds, int64_t rows, int64_t cols,
                                        float* dst, int64_t ldd, int upper) {
  __shared__ float tile[32][33];
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 256 threads: 32 x 8
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = r0 + k, c = c0 + tx;
    tile[k][tx] = (r < rows && c < cols && !(upper && r > c))
                      ? Elem<DT>::load((const typename Elem<DT>::T*)src + r * lds + c)
                      : 0.0f;
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t c = c0 + k, r = r0 + tx;
    if (c < cols && r < rows) dst[c * ldd + r] = tile[tx][k];
  }
}

int launch_transpose_to_f32(hipStream_t s, const void* src, int sdt, int64_t lds, int64_t rows,
                            int64_t cols, float* dst, int64_t ldd, bool upper) {
  if (rows * cols == 0) return IFK_OK;
  if (cdiv(rows, 32) > 65535) {
    set_error("transpose_to_f32: too many rows");
    return IFK_ERR_INVALID;
  }
  const dim3 grid((unsigned)cdiv(cols, 32), (unsigned)cdiv(rows, 32));
  if (sdt == DT_F32)
    hipLaunchKernelGGL(transpose_to_f32_kernel<DT_F32>, grid, dim3(256), 0, s, src, lds, rows, cols,
                       dst, ldd, upper ? 1 : 0);
  else
    hipLaunchKernelGGL(transpose_to_f32_kernel<DT_BF16>, grid, dim3(256), 0, s, src, lds, rows,
                       cols, dst, ldd, upper ? 1 : 0);
  return check_launch("transpose_to_f32");
}

template <int ODT>
__global__ void transpose_upper_kernel(const float* src, int64_t lds, int64_t n, void* out,
                                       int64_t ldo) {
  const int64_t total = n * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / n, j = e % n;
    const float v = (j <= i) ? src[j * lds + i] : 0.0f;
    if constexpr (ODT == DT_F32) ((float*)out)[i * ldo + j] = v;
    else ((bf16_t*)out)[i * ldo + j] = f32_to_bf16(v);
  }
}

int launch_transpose_upper(hipStream_t s, const float* src, int64_t lds, int64_t n, void* out,
                           int odt, int64_t ldo) {
  if (n == 0) return IFK_OK;
  if (odt == DT_F32)
    hipLaunchKernelGGL(transpose_upper_kernel<DT_F32>, dim3(grid_for(n * n)), dim3(256), 0, s, src,
                       lds, n, out, ldo);
  else
    hipLaunchKernelGGL(transpose_upper_kernel<DT_BF16>, dim3(grid_for(n * n)), dim3(256), 0, s, src,
                       lds, n, out, ldo);
  return check_launch("transpose_upper");
}


// out[c][r] (dtype ODT) = src[r][c] for a rows x cols fp32 block, batched over
// blockIdx.z (element strides bss / bso), through a 32 x 32 LDS tile.
template <int ODT>
__global__ void transpose_cast_kernel(const float* src, int64_t lds, int64_t bss, int64_t rows,
                                      int64_t cols, void* out, int64_t ldo, int64_t bso) {
  __shared__ float tile[32][33];
  const float* S = src + (int64_t)blockIdx.z * bss;
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 256 threads: 32 x 8
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = r0 + k, c = c0 + tx;
    tile[k][tx] = (r < rows && c < cols) ? S[r * lds + c] : 0.0f;
  }
  __syncthreads();
  typedef typename Elem<ODT>::T OT;
  OT* O = (OT*)out + (int64_t)blockIdx.z * bso;
  for (int k = ty; k < 32; k += 8) {
    const int64_t c = c0 + k, r = r0 + tx;
    if (c < cols && r < rows) Elem<ODT>::store(O + c * ldo + r, tile[tx][k]);
  }
}

int launch_transpose_cast(hipStream_t s, const float* src, int64_t lds, int64_t rows, int64_t cols,
                          void* out, int odt, int64_t ldo, int batch, int64_t bss, int64_t bso) {
  if (rows * cols == 0 || batch == 0) return IFK_OK;
  if (cdiv(rows, 32) > 65535 || batch > 65535) {
    set_error("transpose_cast: grid too large");
    return IFK_ERR_INVALID;
  }
  const dim3 grid((unsigned)cdiv(cols, 32), (unsigned)cdiv(rows, 32), (unsigned)batch);
  if (odt == DT_F32)
    hipLaunchKernelGGL(transpose_cast_kernel<DT_F32>, grid, dim3(256), 0, s, src, lds, bss, rows,
                       cols, out, ldo, bso);
  else
    hipLaunchKernelGGL(transpose_cast_kernel<DT_BF16>, grid, dim3(256), 0, s, src, lds, bss, rows,
                       cols, out, ldo, bso);
  return check_launch("transpose_cast");
}

// hi[c][r] = RNE bf16(x), lo[c][r] = RNE bf16(x - hi) for x = src[r][c] of a
// rows x cols fp32 block (the bf16 halves of src^T, row stride ldo), through
// a 64 x 64 LDS tile: rows read as float4 when src is 16-byte aligned with
// lds a multiple of 4 (vec_in), the halves written as bf16 pairs when both
// outputs are 4-byte aligned with ldo even (pairs_out).
__global__ __launch_bounds__(256) void split_transpose_kernel(const float* src, int64_t lds,
                                                              int64_t rows, int64_t cols,
                                                              bf16_t* hi, bf16_t* lo, int64_t ldo,
                                                              int vec_in, int pairs_out) {
  __shared__ float tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int t = threadIdx.x;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int rl = (t >> 4) + 16 * q, cl = (t & 15) * 4;
    const int64_t r = r0 + rl, c = c0 + cl;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (r < rows) {
      if (vec_in && c + 3 < cols) {
        const float4 x = *reinterpret_cast<const float4*>(src + r * lds + c);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
      } else {
        for (int u = 0; u < 4; ++u)
          if (c + u < cols) v[u] = src[r * lds + c + u];
      }
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
    const float a = tile[rp][cl], b = tile[rp + 1][cl];
    const bf16_t ah = f32_to_bf16(a), bh = f32_to_bf16(b);
    const bf16_t al = f32_to_bf16(a - bf16_to_f32(ah)), bl = f32_to_bf16(b - bf16_to_f32(bh));
    bf16_t* gh = hi + c * ldo + r;
    bf16_t* gl = lo + c * ldo + r;
    if (pairs_out && r + 1 < rows) {
      *reinterpret_cast<uint32_t*>(gh) = (uint32_t)ah | ((uint32_t)bh << 16);
      *reinterpret_cast<uint32_t*>(gl) = (uint32_t)al | ((uint32_t)bl << 16);
    } else {
      gh[0] = ah;
      gl[0] = al;
      if (r + 1 < rows) {
        gh[1] = bh;
        gl[1] = bl;
      }
    }
  }
}

int launch_split_transpose(hipStream_t s, const float* src, int64_t lds, int64_t rows,
                           int64_t cols, bf16_t* hi, bf16_t* lo, int64_t ldo) {
  if (rows * cols == 0) return IFK_OK;
  if (cdiv(rows, 64) > 65535) {
    set_error("split_transpose: grid too large");
    return IFK_ERR_INVALID;
  }
  const int vec_in = (((uintptr_t)src & 15) == 0) && (lds % 4 == 0);
  const int pairs_out = (((uintptr_t)hi & 3) == 0) && (((uintptr_t)lo & 3) == 0) && (ldo % 2 == 0);
  const dim3 grid((unsigned)cdiv(cols, 64), (unsigned)cdiv(rows, 64));
  hipLaunchKernelGGL(split_transpose_kernel, grid, dim3(256), 0, s, src, lds, rows, cols, hi, lo, ldo,
                     vec_in, pairs_out);
  return check_launch("split_transpose");
}

// dst[c][r] = src[r][c] for a rows x cols bf16 block, through a 64 x 64 LDS
// tile; bf16 pairs move as 32-bit words where both ends of the row are even
// (pair-aligned), element by element otherwise.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const bf16_t* src, int64_t lds,
                                                             int64_t rows, int64_t cols,
                                                             bf16_t* dst, int64_t ldd,
                                                             int pairs_in, int pairs_out) {
  __shared__ bf16_t tile[64][66];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int t = threadIdx.x;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int e = t + 256 * q, r = e >> 5, cp = (e & 31) * 2;
    const int64_t gr = r0 + r, gc = c0 + cp;
    bf16_t a = 0, b = 0;
    if (gr < rows) {
      const bf16_t* g = src + gr * lds + gc;
      if (pairs_in && gc + 1 < cols) {
        const uint32_t w = *(const uint32_t*)g;
        a = (bf16_t)(w & 0xffffu);
        b = (bf16_t)(w >> 16);
      } else {
        if (gc < cols) a = g[0];
        if (gc + 1 < cols) b = g[1];
      }
    }
    tile[r][cp] = a;
    tile[r][cp + 1] = b;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int e = t + 256 * q, c = e >> 5, rp = (e & 31) * 2;
    const int64_t gc = c0 + c, gr = r0 + rp;
    if (gc >= cols) continue;
    bf16_t* g = dst + gc * ldd + gr;
    if (pairs_out && gr + 1 < rows) {
      *(uint32_t*)g = (uint32_t)tile[rp][c] | ((uint32_t)tile[rp + 1][c] << 16);
    } else {
      if (gr < rows) g[0] = tile[rp][c];
      if (gr + 1 < rows) g[1] = tile[rp + 1][c];
    }
  }
}

int launch_transpose_bf16(hipStream_t s, const bf16_t* src, int64_t lds, int64_t rows,
                          int64_t cols, bf16_t* dst, int64_t ldd) {
  if (rows * cols == 0) return IFK_OK;
  if (cdiv(rows, 64) > 65535) {
    set_error("transpose_bf16: grid too large");
    return IFK_ERR_INVALID;
  }
  // pair access needs every row start 4-byte aligned: an even row stride
  // and an aligned base
  const int pin = (lds % 2 == 0) && (((uintptr_t)src & 3) == 0);
  const int pout = (ldd % 2 == 0) && (((uintptr_t)dst & 3) == 0);
  const dim3 grid((unsigned)cdiv(cols, 64), (unsigned)cdiv(rows, 64));
  hipLaunchKernelGGL(transpose_bf16_kernel, grid, dim3(256), 0, s, src, lds, rows, cols, dst, ldd,
                     pin, pout);
  return check_launch("transpose_bf16");
}

// A[i][i] += v for i < n
__global__ void add_diag_kernel(float* A, int64_t lda, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    A[i * lda + i] += v;
}

int launch_add_diag(hipStream_t s, float* A, int64_t lda, int64_t n, float v) {
  if (n <= 0) return IFK_OK;
  hipLaunchKernelGGL(add_diag_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, s, A, lda, n, v);
  return check_launch("add_diag");
}

// S[c][r] = S[r][c] for r > c (the upper triangle from the lower), one 64 x 64
// tile pair per workgroup through LDS: tile (by, bx) with by >= bx is read and
// written transposed into tile (bx, by).  Workgroups of upper tiles exit.
__global__ __launch_bounds__(256) void mirror_lower_kernel(float* S, int64_t ld, int64_t n) {
  if (blockIdx.y < blockIdx.x) return;
  __shared__ float tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int t = threadIdx.x;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int e = t + 256 * q, rl = e >> 6, cl = e & 63;
    const int64_t r = r0 + rl, c = c0 + cl;
    tile[rl][cl] = (r < n && c < n) ? S[r * ld + c] : 0.0f;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int e = t + 256 * q, rl = e >> 6, cl = e & 63;
    // destination (c0 + rl, r0 + cl) holds source (r0 + cl, c0 + rl)
    const int64_t dr = c0 + rl, dc = r0 + cl;
    if (dr < n && dc < n && dc > dr) S[dr * ld + dc] = tile[cl][rl];
  }
}

// Y = alpha X + beta Y (fp32, rows x cols); beta == 0 does not read Y.
__global__ void axpby_kernel(float alpha, const float* X, int64_t ldx, float beta, float* Y,
                             int64_t ldy, int64_t rows, int64_t cols) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / cols, c = e - r * cols;
    const float x = alpha * X[r * ldx + c];
    Y[r * ldy + c] = beta == 0.0f ? x : x + beta * Y[r * ldy + c];
  }
}

int launch_axpby(hipStream_t s, float alpha, const float* X, int64_t ldx, float beta, float* Y,
                 int64_t ldy, int64_t rows, int64_t cols) {
  if (rows * cols <= 0) return IFK_OK;
  const int64_t blocks = std::min<int64_t>(cdiv(rows * cols, 256), 65536);
  hipLaunchKernelGGL(axpby_kernel, dim3((unsigned)blocks), dim3(256), 0, s, alpha, X, ldx, beta,
                     Y, ldy, rows, cols);
  return check_launch("axpby");
}

int launch_mirror_lower(hipStream_t s, float* S, int64_t ld, int64_t n) {
  if (n <= 0) return IFK_OK;
  if (cdiv(n, 64) > 65535) {
    set_error("mirror_lower: matrix too large");
    return IFK_ERR_INVALID;
  }
  const dim3 grid((unsigned)cdiv(n, 64), (unsigned)cdiv(n, 64));
  hipLaunchKernelGGL(mirror_lower_kernel, grid, dim3(256), 0, s, S, ld, n);
  return check_launch("mirror_lower");
}


// ---------------------------------------------------------------------------
// Power-iteration helpers of the condition estimate (linalg.hip: cond_est).
// ---------------------------------------------------------------------------

// V (n x k, row-major) <- deterministic probe vectors: hashed values in
// [-1, 1), column 0 shifted by +1 so that it overlaps a dominant direction
// with all-positive weights (the mean of a layer's activations).
__global__ void probe_init_kernel(float* V, int64_t n, int k) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n * k;
       e += (int64_t)gridDim.x * blockDim.x) {
    uint32_t h = (uint32_t)e * 2654435761u + 0x9e3779b9u;
    h ^= h >> 16;
    h *= 0x85ebca6bu;
    h ^= h >> 13;
    h *= 0xc2b2ae35u;
    h ^= h >> 16;
    const float u = (float)(h >> 8) * (1.0f / 8388608.0f) - 1.0f;
    V[e] = u + ((e % k) == 0 ? 1.0f : 0.0f);
  }
}

// Column j of V (n x k) scaled to unit norm (left alone if zero or not
// finite); its sum of squares before scaling into ss[j].  One workgroup per
// column.
__global__ __launch_bounds__(256) void colnorm_kernel(float* V, int64_t n, int k, float* ss) {
  __shared__ float red[256];
  const int j = blockIdx.x;
  float acc = 0.0f;
  for (int64_t i = threadIdx.x; i < n; i += 256) {
    const float v = V[i * k + j];
    acc = fmaf(v, v, acc);
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  const float tot = red[0];
  if (threadIdx.x == 0) ss[j] = tot;
  if (!(tot > 0.0f) || !isfinite(tot)) return;
  const float sc = 1.0f / sqrtf(tot);
  for (int64_t i = threadIdx.x; i < n; i += 256) V[i * k + j] *= sc;
}

// kappa = (max_j ssa[j] * max_j ssb[j])^(1/4): each max is the squared norm
// of M^T M v for a unit v, about sigma_max(M)^4.
__global__ void cond_final_kernel(const float* ssa, const float* ssb, int k, float* kappa) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  float a = 0.0f, b = 0.0f;
  for (int j = 0; j < k; ++j) {
    a = fmaxf(a, ssa[j]);
    b = fmaxf(b, ssb[j]);
  }
  *kappa = sqrtf(sqrtf(a) * sqrtf(b));
}

int launch_probe_init(hipStream_t s, float* V, int64_t n, int k) {
  hipLaunchKernelGGL(probe_init_kernel, dim3(grid_for(n * k)), dim3(256), 0, s, V, n, k);
  return check_launch("probe_init");
}

int launch_colnorm(hipStream_t s, float* V, int64_t n, int k, float* ss) {
  hipLaunchKernelGGL(colnorm_kernel, dim3((unsigned)k), dim3(256), 0, s, V, n, k, ss);
  return check_launch("colnorm");
}

int launch_cond_final(hipStream_t s, const float* ssa, const float* ssb, int k, float* kappa) {
  hipLaunchKernelGGL(cond_final_kernel, dim3(1), dim3(64), 0, s, ssa, ssb, k, kappa);
  return check_launch("cond_final");
}

}  // namespace ifk
