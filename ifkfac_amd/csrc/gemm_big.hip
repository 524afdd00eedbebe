// Large-tile bf16 MFMA GEMM for the big contractions of the curvature path
// (block-reflector updates of the fold, preconditioning products).
//
// Block tile 256 x 128 x 32, 256 threads = 4 waves in a 2 x 2 grid, each wave
// owning a 128 x 64 sub-tile as 4 x 2 v_mfma_f32_32x32x16_bf16 accumulators
// (128 fp32 accumulator registers per lane).  Two workgroups fit a CU
// (registers and LDS), so one hides the other's memory latency.  Operands are
// staged global -> registers -> LDS, converted to bf16 with the hardware RNE
// conversion on the way; the LDS holds two K slabs (double buffer), so one
// workgroup barrier per 32-wide K step separates "store slab k+1" from
// "read slab k".  In LDS both operands are K-contiguous per row (row stride
// 40 bf16 = 80 bytes), so each lane reads its 8-element MFMA fragment with one
// 128-bit load; operands that are K-strided in memory are transposed in
// registers (8 k x 2 mn per thread).  Contract and operand conventions:
// gemm.h.  The 256 x 128 tile reads 85 flops per operand byte from L2 at
// bf16 (43 at fp32), against 64 / 32 for the 128 x 128 engine of gemm.hip.
#include "gemm_impl.h"

namespace ifk {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 128, BK = 32, NTH = 256;
constexpr int LW = BK + 8;  // LDS row stride in bf16 elements

__device__ inline uint32_t cvt2(float lo, float hi) {
  bf16x2_t v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

template <int DT>
__device__ inline float ld1(const void* base, int64_t idx) {
  if constexpr (DT == DT_F32) return ((const float*)base)[idx];
  else return bf16_to_f32(((const bf16_t*)base)[idx]);
}

// Structural zero of a triangular operand (see gemm.h): for A, mn = m of
// op(A)[m][k]; for B, mn = n of op(B)[k][n].
template <bool ISA>
__device__ inline bool tri0(int tri, int64_t mn, int64_t k) {
  if (tri == TRI_NONE) return false;
  if constexpr (ISA) return tri == TRI_UPPER ? (k < mn) : (k > mn);
  else return tri == TRI_UPPER ? (k > mn) : (k < mn);
}

// Operand slab ROWS (mn) x 32 (k) of one operand in flight: RW raw 32-bit
// registers per thread (fp32 values, or bf16 pairs as stored in memory).
// load() only issues the loads (the values are consumed after the MFMAs of
// the current slab, so the loads overlap them); put() converts to bf16 pairs
// along k (RNE) and writes the slab to LDS.  Thread mapping:
//   K-contiguous: group q covers row mn = (t + NTH q) / 4, k = 8 ((t + NTH q) % 4) + e
//   MN-contiguous: job u = t + NTH u' covers mn = 2 (u % (ROWS / 2)) + j,
//                  k = 8 (u / (ROWS / 2)) + e
template <int DT, int ROWS>
struct Slab {
  static constexpr int RW = DT == DT_F32 ? ROWS / 8 : ROWS / 16;
  uint32_t r[RW];
  bool fast;
};

// Does the 32-wide K slab starting at k0 cross the structural-zero triangle of
// a triangular operand over its rows [mn0, mn0 + ROWS)?  Only such slabs are
// masked element by element (see tri0).
template <bool ISA, int ROWS>
__device__ inline bool slab_crosses(int tri, int64_t mn0, int64_t k0) {
  if (tri == TRI_NONE) return false;
  const bool zero_low_k = ISA ? tri == TRI_UPPER : tri == TRI_LOWER;  // zero where k < mn
  return zero_low_k ? (k0 < mn0 + ROWS - 1) : (k0 + BK - 1 > mn0);
}

template <int DT, bool KC, bool ISA, int ROWS>
__device__ inline void load(Slab<DT, ROWS>& S, const void* base, int64_t ld, int64_t MN, int64_t K,
                            int64_t mn0, int64_t k0, int tri, bool vec, int t) {
  S.fast = vec && (mn0 + ROWS <= MN) && (k0 + BK <= K);
  if (S.fast) {
    if constexpr (KC) {
#pragma unroll
      for (int q = 0; q < ROWS / 64; ++q) {
        const int g = t + NTH * q;
        const int64_t idx = (mn0 + (g >> 2)) * ld + k0 + (g & 3) * 8;
        if constexpr (DT == DT_F32) {
          const uint4* p4 = (const uint4*)((const float*)base + idx);
          const uint4 a = p4[0], b = p4[1];
          S.r[8 * q + 0] = a.x; S.r[8 * q + 1] = a.y; S.r[8 * q + 2] = a.z; S.r[8 * q + 3] = a.w;
          S.r[8 * q + 4] = b.x; S.r[8 * q + 5] = b.y; S.r[8 * q + 6] = b.z; S.r[8 * q + 7] = b.w;
        } else {
          const uint4 w = *(const uint4*)((const bf16_t*)base + idx);
          S.r[4 * q + 0] = w.x; S.r[4 * q + 1] = w.y; S.r[4 * q + 2] = w.z; S.r[4 * q + 3] = w.w;
        }
      }
    } else {
#pragma unroll
      for (int u2 = 0; u2 < ROWS / 128; ++u2) {
        const int jid = t + NTH * u2;
        const int64_t idx = (k0 + 8 * (jid / (ROWS / 2))) * ld + mn0 + 2 * (jid % (ROWS / 2));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if constexpr (DT == DT_F32) {
            const uint2 a = *(const uint2*)((const float*)base + idx + e * ld);
            S.r[16 * u2 + e] = a.x;        // mn
            S.r[16 * u2 + 8 + e] = a.y;    // mn + 1
          } else {
            S.r[8 * u2 + e] = *(const uint32_t*)((const bf16_t*)base + idx + e * ld);
          }
        }
      }
    }
    return;
  }
  // Edges and triangular operands: guarded element loads, kept as fp32 bits
  // (bf16 operands are widened; their RW registers hold bf16 pairs instead).
  if constexpr (KC) {
#pragma unroll
    for (int q = 0; q < ROWS / 64; ++q) {
      const int g = t + NTH * q;
      const int64_t gm = mn0 + (g >> 2), gk = k0 + (g & 3) * 8;
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        f[e] = (gm < MN && gk + e < K) ? ld1<DT>(base, gm * ld + gk + e) : 0.0f;
        if (tri0<ISA>(tri, gm, gk + e)) f[e] = 0.0f;
      }
      if constexpr (DT == DT_F32) {
#pragma unroll
        for (int e = 0; e < 8; ++e) S.r[8 * q + e] = __float_as_uint(f[e]);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) S.r[4 * q + c] = cvt2(f[2 * c], f[2 * c + 1]);
      }
    }
  } else {
#pragma unroll
    for (int u2 = 0; u2 < ROWS / 128; ++u2) {
      const int jid = t + NTH * u2;
      const int64_t gm = mn0 + 2 * (jid % (ROWS / 2));
      const int64_t kb = k0 + 8 * (jid / (ROWS / 2));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t gk = kb + e;
        float f0 = (gm < MN && gk < K) ? ld1<DT>(base, gk * ld + gm) : 0.0f;
        float f1 = (gm + 1 < MN && gk < K) ? ld1<DT>(base, gk * ld + gm + 1) : 0.0f;
        if (tri0<ISA>(tri, gm, gk)) f0 = 0.0f;
        if (tri0<ISA>(tri, gm + 1, gk)) f1 = 0.0f;
        if constexpr (DT == DT_F32) {
          S.r[16 * u2 + e] = __float_as_uint(f0);
          S.r[16 * u2 + 8 + e] = __float_as_uint(f1);
        } else {
          S.r[8 * u2 + e] = cvt2(f0, f1);   // same layout as the memory pair (mn, mn + 1)
        }
      }
    }
  }
}

template <int DT, bool KC, bool ISA, int ROWS>
__device__ inline void put(bf16_t* L, const Slab<DT, ROWS>& S, int t, int tri, int64_t mn0,
                           int64_t k0) {
  // fast slabs that cross the triangle are masked here (the edge path masked
  // on load)
  const bool mask = S.fast && slab_crosses<ISA, ROWS>(tri, mn0, k0);
#pragma unroll
  for (int q = 0; q < ROWS / 64; ++q) {
    int mn, kk;
    uint32_t w[4];
    if constexpr (KC) {
      const int g = t + NTH * q;
      mn = g >> 2;
      kk = (g & 3) * 8;
      if constexpr (DT == DT_F32) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          w[c] = cvt2(__uint_as_float(S.r[8 * q + 2 * c]), __uint_as_float(S.r[8 * q + 2 * c + 1]));
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) w[c] = S.r[4 * q + c];
      }
    } else {
      const int u2 = q >> 1, j = q & 1;
      const int jid = t + NTH * u2;
      mn = 2 * (jid % (ROWS / 2)) + j;
      kk = 8 * (jid / (ROWS / 2));
      if constexpr (DT == DT_F32) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          w[c] = cvt2(__uint_as_float(S.r[16 * u2 + 8 * j + 2 * c]),
                      __uint_as_float(S.r[16 * u2 + 8 * j + 2 * c + 1]));
      } else {
        // memory pairs (mn, mn + 1) at k = 2c and 2c + 1 -> k pairs of one mn
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t a = S.r[8 * u2 + 2 * c], b = S.r[8 * u2 + 2 * c + 1];
          w[c] = j == 0 ? ((a & 0xffffu) | (b << 16)) : ((a >> 16) | (b & 0xffff0000u));
        }
      }
    }
    if (mask) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (tri0<ISA>(tri, mn0 + mn, k0 + kk + 2 * c)) w[c] &= 0xffff0000u;
        if (tri0<ISA>(tri, mn0 + mn, k0 + kk + 2 * c + 1)) w[c] &= 0x0000ffffu;
      }
    }
    *(uint4*)(&L[mn * LW + kk]) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// One output tile (tile index `tile` of grid z) of the product.
template <int ADT, bool AKC, int BDT, bool BKC>
__device__ __forceinline__ void gemm_big_tile(const GemmParams& p, int tile, bf16_t (&As)[2][BM * LW],
                                              bf16_t (&Bs)[2][BN * LW]) {
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, h = lane >> 5;
  const int tm = tile % p.tiles_m, tn = tile / p.tiles_m;
  const int z = blockIdx.z;
  const int bidx = z / p.splits, split = z % p.splits;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  if (p.upper_only && m0 >= n0 + BN) return;   // wholly below the diagonal
  if (p.lower_only && n0 >= m0 + BM) return;   // wholly above the diagonal
  const void* Ab = (const char*)p.A + (size_t)bidx * p.bsa * (ADT == DT_F32 ? 4 : 2);
  const void* Bb = (const char*)p.B + (size_t)bidx * p.bsb * (BDT == DT_F32 ? 4 : 2);

  int64_t klo = 0, khi = p.K;
  if (p.tria == TRI_UPPER) klo = max(klo, m0);
  if (p.tria == TRI_LOWER) khi = min(khi, m0 + BM);
  if (p.trib == TRI_UPPER) khi = min(khi, n0 + BN);
  if (p.trib == TRI_LOWER) klo = max(klo, n0);
  klo = klo / BK * BK;
  const int64_t nkt = khi > klo ? (khi - klo + BK - 1) / BK : 0;
  const int64_t per = (nkt + p.splits - 1) / p.splits;
  const int64_t kt0 = (int64_t)split * per;
  const int64_t kt1 = min(nkt, kt0 + per);

  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  Slab<ADT, BM> sa;
  Slab<BDT, BN> sb;
  if (kt0 < kt1) {
    const int64_t k0 = klo + kt0 * BK;
    load<ADT, AKC, true, BM>(sa, Ab, p.lda, p.M, khi, m0, k0, p.tria, p.vec_a, t);
    load<BDT, BKC, false, BN>(sb, Bb, p.ldb, p.N, khi, n0, k0, p.trib, p.vec_b, t);
    put<ADT, AKC, true, BM>(As[0], sa, t, p.tria, m0, k0);
    put<BDT, BKC, false, BN>(Bs[0], sb, t, p.trib, n0, k0);
  }
  __syncthreads();
  for (int64_t kt = kt0; kt < kt1; ++kt) {
    const int cur = (int)((kt - kt0) & 1);
    const bool more = kt + 1 < kt1;
    if (more) {  // loads of slab k+1 overlap the MFMAs of slab k
      const int64_t k0 = klo + (kt + 1) * BK;
      load<ADT, AKC, true, BM>(sa, Ab, p.lda, p.M, khi, m0, k0, p.tria, p.vec_a, t);
      load<BDT, BKC, false, BN>(sb, Bb, p.ldb, p.N, khi, n0, k0, p.trib, p.vec_b, t);
    }
    const bf16_t* Ac = As[cur];
    const bf16_t* Bc = Bs[cur];
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t af[4], bfr[2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *(const bf16x8_t*)(&Ac[(wm * 128 + i * 32 + l32) * LW + ks * 16 + h * 8]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bfr[j] = *(const bf16x8_t*)(&Bc[(wn * 64 + j * 32 + l32) * LW + ks * 16 + h * 8]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      const int64_t k0 = klo + (kt + 1) * BK;
      put<ADT, AKC, true, BM>(As[cur ^ 1], sa, t, p.tria, m0, k0);
      put<BDT, BKC, false, BN>(Bs[cur ^ 1], sb, t, p.trib, n0, k0);
    }
    __syncthreads();
  }

  // acc[i][j][r]: row (r / 4) * 8 + h * 4 + r % 4, column l32 of 32 x 32 tile (i, j)
  if (p.splits > 1) {
    float* P = p.part + ((size_t)(bidx * p.splits + split)) * (size_t)p.M * (size_t)p.N;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * 128 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
          const int64_t col = n0 + wn * 64 + j * 32 + l32;
          if (row < p.M && col < p.N) P[row * p.N + col] = acc[i][j][r];
        }
    return;
  }
  float* Cp = p.C ? p.C + (size_t)bidx * p.bsc : nullptr;
  bf16_t* Cbp = p.Cb ? p.Cb + (size_t)bidx * p.bscb : nullptr;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn * 64 + j * 32 + l32;
      float old[16];
      if (p.beta != 0.0f) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * 128 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
          old[r] = (row < p.M && col < p.N) ? Cp[row * p.ldc + col] : 0.0f;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * 128 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
        if (row < p.M && col < p.N) {
          float v = p.alpha * acc[i][j][r];
          if (p.beta != 0.0f) v += p.beta * old[r];
          if (Cp) Cp[row * p.ldc + col] = v;
          if (Cbp) Cbp[row * p.ldcb + col] = f32_to_bf16(v);
        }
      }
    }
}

// Tiles are visited grid-stride, so a launch may use fewer workgroups than
// tiles (leaving CUs to kernels on other streams).
template <int ADT, bool AKC, int BDT, bool BKC>
__global__ __launch_bounds__(NTH, 2) void gemm_big_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) bf16_t As[2][BM * LW];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][BN * LW];
  const int tiles = p.tiles_m * p.tiles_n;
  for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    gemm_big_tile<ADT, AKC, BDT, BKC>(p, tile, As, Bs);
    __syncthreads();   // the LDS slabs are reused by the next tile
  }
}

template <int ADT, bool AKC, int BDT, bool BKC>
void launch_t(hipStream_t s, dim3 g, const GemmParams& p) {
  hipLaunchKernelGGL((gemm_big_kernel<ADT, AKC, BDT, BKC>), g, dim3(NTH), 0, s, p);
}

template <int ADT, bool AKC>
void launch_b(hipStream_t s, dim3 g, const GemmParams& p, int bdt, bool bkc) {
  if (bdt == DT_F32) {
    if (bkc) launch_t<ADT, AKC, DT_F32, true>(s, g, p);
    else launch_t<ADT, AKC, DT_F32, false>(s, g, p);
  } else {
    if (bkc) launch_t<ADT, AKC, DT_BF16, true>(s, g, p);
    else launch_t<ADT, AKC, DT_BF16, false>(s, g, p);
  }
}

}  // namespace

int gemm_big_tile_m() { return BM; }
int gemm_big_tile_n() { return BN; }
int gemm_big_bk() { return BK; }

void launch_gemm_big(hipStream_t s, dim3 grid, const GemmParams& p, int adt, bool akc, int bdt,
                     bool bkc) {
  if (adt == DT_F32) {
    if (akc) launch_b<DT_F32, true>(s, grid, p, bdt, bkc);
    else launch_b<DT_F32, false>(s, grid, p, bdt, bkc);
  } else {
    if (akc) launch_b<DT_BF16, true>(s, grid, p, bdt, bkc);
    else launch_b<DT_BF16, false>(s, grid, p, bdt, bkc);
  }
}

}  // namespace ifk
