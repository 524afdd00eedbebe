// MFMA GEMM engine (gfx950).  Contract in gemm.h.
//
// Block tile 128 x 128, 256 threads = 4 waves in a 2 x 2 grid, each wave owns a
// 64 x 64 sub-tile computed as 2 x 2 MFMA 32x32 tiles (4 f32x16 accumulators).
// K is staged through LDS in slabs of BK (64 for bf16, 32 for fp32) with a
// register prefetch of the next slab while the current one feeds the MFMAs.
// In LDS both operands are stored K-contiguous per row so every lane reads its
// MFMA fragment with 128-bit loads; operands that are K-strided in memory are
// transposed in registers on the way in (8 k x 4 mn micro-blocks per thread).
#include "gemm_impl.h"
#include "kernels.h"

#include <mutex>
#include <vector>

namespace ifk {

// ---------------------------------------------------------------------------
// Opt-in launch profiler: when armed for a GEMM variant (or for all), each
// launch of that variant is bracketed by a pair of HIP events recorded on the
// launching stream, and its algorithmic flops and bytes are kept.  Disarmed,
// the cost is one integer compare per GEMM call.
// ---------------------------------------------------------------------------
struct ProfRec {
  hipEvent_t beg, end;
  int variant;
  int64_t m, n, k;
  double flops, bytes;
};

static std::mutex g_prof_mu;
static int g_prof_variant = -1;  // -1 off, -2 all variants
static std::vector<ProfRec> g_prof;
static size_t g_prof_used = 0;

int gemm_variant_id(int math, int adt, bool akc, int bdt, bool bkc) {
  return (math << 4) | (adt << 3) | ((akc ? 1 : 0) << 2) | (bdt << 1) | (bkc ? 1 : 0);
}

int profile_begin(int variant) {
  std::lock_guard<std::mutex> g(g_prof_mu);
  g_prof_variant = variant;
  g_prof_used = 0;
  return IFK_OK;
}

int profile_end(int64_t* n_launches) {
  std::lock_guard<std::mutex> g(g_prof_mu);
  g_prof_variant = -1;
  for (size_t i = 0; i < g_prof_used; ++i) {
    if (hipEventSynchronize(g_prof[i].end) != hipSuccess) {
      set_error("profile_end: event synchronisation failed");
      return IFK_ERR_HIP;
    }
  }
  if (n_launches) *n_launches = (int64_t)g_prof_used;
  return IFK_OK;
}

int profile_get(int64_t i, int* variant, float* ms, double* flops, double* bytes, int64_t* m,
                int64_t* n, int64_t* k) {
  std::lock_guard<std::mutex> g(g_prof_mu);
  if (i < 0 || (size_t)i >= g_prof_used) {
    set_error("profile_get: index out of range");
    return IFK_ERR_INVALID;
  }
  const ProfRec& r = g_prof[i];
  float t = 0.0f;
  if (hipEventElapsedTime(&t, r.beg, r.end) != hipSuccess) {
    set_error("profile_get: elapsed time unavailable");
    return IFK_ERR_HIP;
  }
  *variant = r.variant;
  *ms = t;
  *flops = r.flops;
  *bytes = r.bytes;
  *m = r.m;
  *n = r.n;
  *k = r.k;
  return IFK_OK;
}

// Kernel family of a variant id: 0 the 128 x 128 kernel, 1 the 256 x 128
// register-staged kernel (bit 5), 2 / 3 the direct-to-LDS kernel with its 256
// / 128 tile (bits 5 and 6, and bit 7 for the 128 tile; bit 9 marks a
// stream-K launch of either).
static int gemm_family(int vid) {
  if (vid >= KVID) return 5 + (vid - KVID);   // 5 cholb_first, 6 cholb_step
  if ((vid >> 6) & 1) return ((vid >> 7) & 1) ? 3 : 2;
  return (vid >> 5) & 1;
}

// Armed variant: >= 0 one variant id, -2 every launch, -3 / -4 / -5 / -6 /
// -7 / -8 every launch of family 1 / 0 / 2 / 3 / 5 / 6.
static ProfRec* prof_slot(int vid) {
  const int a = g_prof_variant;
  if (a == -1) return nullptr;
  if (a >= 0 && a != vid) return nullptr;
  const int fam = gemm_family(vid);
  if ((a == -3 && fam != 1) || (a == -4 && fam != 0) || (a == -5 && fam != 2) ||
      (a == -6 && fam != 3) || (a == -7 && fam != 5) || (a == -8 && fam != 6))
    return nullptr;
  std::lock_guard<std::mutex> g(g_prof_mu);
  if (g_prof_used == g_prof.size()) {
    ProfRec r{};
    if (hipEventCreate(&r.beg) != hipSuccess || hipEventCreate(&r.end) != hipSuccess)
      return nullptr;
    g_prof.push_back(r);
  }
  return &g_prof[g_prof_used++];
}

void* prof_kernel_begin(hipStream_t s, int vid, double flops, double bytes, int64_t m, int64_t n,
                        int64_t k) {
  ProfRec* pr = prof_slot(vid);
  if (!pr) return nullptr;
  pr->variant = vid;
  pr->m = m;
  pr->n = n;
  pr->k = k;
  pr->flops = flops;
  pr->bytes = bytes;
  hipEventRecord(pr->beg, s);
  return pr;
}

void prof_kernel_end(void* rec, hipStream_t s) {
  if (rec) hipEventRecord(static_cast<ProfRec*>(rec)->end, s);
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int GBM = 128;
constexpr int GBN = 128;
constexpr int GNT = 256;

template <int MATH> struct GCfg;
template <> struct GCfg<MATH_BF16> {
  static constexpr int BK = 64;
  static constexpr int LDW = 72;  // LDS row stride in elements (bf16)
  static constexpr int G = 8;     // k values per staged group
  typedef bf16_t LT;
};
template <> struct GCfg<MATH_F32> {
  static constexpr int BK = 32;
  static constexpr int LDW = 36;  // LDS row stride in elements (fp32)
  static constexpr int G = 4;
  typedef float LT;
};

template <int DT>
__device__ inline float ld_elem(const void* base, int64_t idx) {
  if constexpr (DT == DT_F32) {
    return ((const float*)base)[idx];
  } else {
    return bf16_to_f32(((const bf16_t*)base)[idx]);
  }
}

// Load `cnt` (4 or 8) consecutive elements starting at base[idx] as floats.
// Caller guarantees alignment (idx multiple of cnt, base 16-byte aligned).
template <int DT, int CNT>
__device__ inline void ld_vec(const void* base, int64_t idx, float* out) {
  if constexpr (DT == DT_F32) {
    const float4* p = (const float4*)((const float*)base + idx);
#pragma unroll
    for (int c = 0; c < CNT / 4; ++c) {
      float4 v = p[c];
      out[4 * c + 0] = v.x; out[4 * c + 1] = v.y; out[4 * c + 2] = v.z; out[4 * c + 3] = v.w;
    }
  } else {
    const bf16_t* b = (const bf16_t*)base + idx;
    if constexpr (CNT == 8) {
      uint4 v = *(const uint4*)b;
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        out[2 * c] = bf16_to_f32((bf16_t)(w[c] & 0xffffu));
        out[2 * c + 1] = bf16_to_f32((bf16_t)(w[c] >> 16));
      }
    } else {
      uint2 v = *(const uint2*)b;
      uint32_t w[2] = {v.x, v.y};
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        out[2 * c] = bf16_to_f32((bf16_t)(w[c] & 0xffffu));
        out[2 * c + 1] = bf16_to_f32((bf16_t)(w[c] >> 16));
      }
    }
  }
}

// Is element (mn, k) of the operand structurally zero?  For A, mn = m of
// op(A)[m][k]; for B, mn = n of op(B)[k][n].
template <bool ISA>
__device__ inline bool tri_zero(int tri, int64_t mn, int64_t k) {
  if (tri == TRI_NONE) return false;
  if constexpr (ISA) {
    return tri == TRI_UPPER ? (k < mn) : (k > mn);
  } else {
    return tri == TRI_UPPER ? (k > mn) : (k < mn);
  }
}

// Stage one operand slab (128 rows of mn x BK k values) into registers as 4
// groups of G consecutive k values each.
template <int MATH, int DT, bool KC, bool ISA>
__device__ inline void stage_load(float (&v)[4][GCfg<MATH>::G], const void* base, int64_t ld,
                                  int64_t MN, int64_t K, int64_t mn0, int64_t k0, int tri,
                                  bool vec, int t) {
  constexpr int G = GCfg<MATH>::G;
  constexpr int BK = GCfg<MATH>::BK;
  const bool interior = vec && (mn0 + 128 <= MN) && (k0 + BK <= K);
  if constexpr (KC) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int g = t + GNT * q;
      const int mn = g / (BK / G);
      const int kk = (g % (BK / G)) * G;
      const int64_t gm = mn0 + mn, gk = k0 + kk;
      if (interior) {
        ld_vec<DT, G>(base, gm * ld + gk, v[q]);
      } else {
#pragma unroll
        for (int e = 0; e < G; ++e) {
          v[q][e] = (gm < MN && gk + e < K) ? ld_elem<DT>(base, gm * ld + gk + e) : 0.0f;
        }
      }
      if (tri != TRI_NONE) {
#pragma unroll
        for (int e = 0; e < G; ++e)
          if (tri_zero<ISA>(tri, gm, gk + e)) v[q][e] = 0.0f;
      }
    }
  } else {
    // micro-block: G k values x 4 mn values per thread
    const int mnb = (t & 31) * 4;
    const int kb = (t >> 5) * G;
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int64_t gk = k0 + kb + i;
      float w[4];
      if (interior) {
        ld_vec<DT, 4>(base, gk * ld + mn0 + mnb, w);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t gm = mn0 + mnb + j;
          w[j] = (gm < MN && gk < K) ? ld_elem<DT>(base, gk * ld + gm) : 0.0f;
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j][i] = w[j];
    }
    if (tri != TRI_NONE) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < G; ++i)
          if (tri_zero<ISA>(tri, mn0 + mnb + j, k0 + kb + i)) v[j][i] = 0.0f;
    }
  }
}

// Write staged groups into the LDS slab (row-major [mn][k], K contiguous).
template <int MATH, bool KC>
__device__ inline void stage_store(typename GCfg<MATH>::LT* Xs, const float (&v)[4][GCfg<MATH>::G],
                                   int t) {
  constexpr int G = GCfg<MATH>::G;
  constexpr int BK = GCfg<MATH>::BK;
  constexpr int LDW = GCfg<MATH>::LDW;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int mn, kk;
    if constexpr (KC) {
      const int g = t + GNT * q;
      mn = g / (BK / G);
      kk = (g % (BK / G)) * G;
    } else {
      mn = (t & 31) * 4 + q;
      kk = (t >> 5) * G;
    }
    if constexpr (MATH == MATH_BF16) {
      uint4 w;
      w.x = pack_bf16x2(v[q][0], v[q][1]);
      w.y = pack_bf16x2(v[q][2], v[q][3]);
      w.z = pack_bf16x2(v[q][4], v[q][5]);
      w.w = pack_bf16x2(v[q][6], v[q][7]);
      *(uint4*)(&Xs[mn * LDW + kk]) = w;
    } else {
      // fp32 slab keeps even k in positions 0..15 and odd k in 16..31 so that a
      // lane's operands for consecutive 32x32x2 steps are contiguous.
      float* row = (float*)Xs + mn * LDW;
      *(float2*)(&row[kk / 2]) = make_float2(v[q][0], v[q][2]);
      *(float2*)(&row[16 + kk / 2]) = make_float2(v[q][1], v[q][3]);
    }
  }
}

template <int MATH, int ADT, bool AKC, int BDT, bool BKC>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
  constexpr int BK = GCfg<MATH>::BK;
  constexpr int LDW = GCfg<MATH>::LDW;
  constexpr int G = GCfg<MATH>::G;
  typedef typename GCfg<MATH>::LT LT;
  __shared__ __attribute__((aligned(16))) LT As[GBM * LDW];
  __shared__ __attribute__((aligned(16))) LT Bs[GBN * LDW];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int tile = blockIdx.x;
  const int tm = tile % p.tiles_m, tn = tile / p.tiles_m;
  const int z = blockIdx.z;
  const int bidx = z / p.splits, split = z % p.splits;
  const int64_t m0 = (int64_t)tm * GBM, n0 = (int64_t)tn * GBN;
  if (p.upper_only && m0 >= n0 + GBN) return;   // wholly below the diagonal
  if (p.lower_only && n0 >= m0 + GBM) return;   // wholly above the diagonal

  const void* Ab = (const char*)p.A + (size_t)bidx * p.bsa * (ADT == DT_F32 ? 4 : 2);
  const void* Bb = (const char*)p.B + (size_t)bidx * p.bsb * (BDT == DT_F32 ? 4 : 2);

  // K range of this tile after triangular structure, then this split's share.
  int64_t klo = 0, khi = p.K;
  if (p.tria == TRI_UPPER) klo = max(klo, m0);
  if (p.tria == TRI_LOWER) khi = min(khi, m0 + GBM);
  if (p.trib == TRI_UPPER) khi = min(khi, n0 + GBN);
  if (p.trib == TRI_LOWER) klo = max(klo, n0);
  int64_t nkt = khi > klo ? (khi - klo + BK - 1) / BK : 0;
  int64_t per = (nkt + p.splits - 1) / p.splits;
  int64_t kt0 = (int64_t)split * per;
  int64_t kt1 = min(nkt, kt0 + per);

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  float va[4][G], vb[4][G];
  if (kt0 < kt1) {
    stage_load<MATH, ADT, AKC, true>(va, Ab, p.lda, p.M, khi, m0, klo + kt0 * BK, p.tria,
                                     p.vec_a, t);
    stage_load<MATH, BDT, BKC, false>(vb, Bb, p.ldb, p.N, khi, n0, klo + kt0 * BK, p.trib,
                                      p.vec_b, t);
  }
  const int h = lane >> 5;
  const int l32 = lane & 31;
  for (int64_t kt = kt0; kt < kt1; ++kt) {
    stage_store<MATH, AKC>(As, va, t);
    stage_store<MATH, BKC>(Bs, vb, t);
    __syncthreads();
    if (kt + 1 < kt1) {
      const int64_t kn = klo + (kt + 1) * BK;
      stage_load<MATH, ADT, AKC, true>(va, Ab, p.lda, p.M, khi, m0, kn, p.tria, p.vec_a, t);
      stage_load<MATH, BDT, BKC, false>(vb, Bb, p.ldb, p.N, khi, n0, kn, p.trib, p.vec_b, t);
    }
    if constexpr (MATH == MATH_BF16) {
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        bf16x8_t af[2], bfr[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
          af[i] = *(const bf16x8_t*)(&As[(wm * 64 + i * 32 + l32) * LDW + ks * 16 + h * 8]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          bfr[j] = *(const bf16x8_t*)(&Bs[(wn * 64 + j * 32 + l32) * LDW + ks * 16 + h * 8]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      }
    } else {
      float af[2][16], bfr[2][16];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float* row = (const float*)As + (wm * 64 + i * 32 + l32) * LDW + h * 16;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float4 v = *(const float4*)(row + 4 * c);
          af[i][4 * c] = v.x; af[i][4 * c + 1] = v.y; af[i][4 * c + 2] = v.z; af[i][4 * c + 3] = v.w;
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float* row = (const float*)Bs + (wn * 64 + j * 32 + l32) * LDW + h * 16;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float4 v = *(const float4*)(row + 4 * c);
          bfr[j][4 * c] = v.x; bfr[j][4 * c + 1] = v.y; bfr[j][4 * c + 2] = v.z; bfr[j][4 * c + 3] = v.w;
        }
      }
#pragma unroll
      for (int s = 0; s < 16; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bfr[j][s], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // Epilogue.  acc[i][j][r] holds row (r/4)*8 + h*4 + r%4, column l32 of the
  // 32x32 tile (i, j) of this wave.
  if (p.splits > 1) {
    float* P = p.part + ((size_t)(bidx * p.splits + split)) * (size_t)p.M * (size_t)p.N;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
          const int64_t col = n0 + wn * 64 + j * 32 + l32;
          if (row < p.M && col < p.N) P[row * p.N + col] = acc[i][j][r];
        }
    return;
  }
  float* Cp = p.C ? p.C + (size_t)bidx * p.bsc : nullptr;
  bf16_t* Cbp = p.Cb ? p.Cb + (size_t)bidx * p.bscb : nullptr;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
        const int64_t col = n0 + wn * 64 + j * 32 + l32;
        if (row < p.M && col < p.N) {
          float v = p.alpha * acc[i][j][r];
          if (p.beta != 0.0f) v += p.beta * Cp[row * p.ldc + col];
          if (Cp) Cp[row * p.ldc + col] = v;
          if (Cbp) Cbp[row * p.ldcb + col] = f32_to_bf16(v);
        }
      }
}

__global__ void splitk_reduce_kernel(GemmParams p) {
  const int64_t MN = p.M * p.N;
  const int bidx = blockIdx.y;
  const float* P = p.part + (size_t)bidx * p.splits * MN;
  float* Cp = p.C ? p.C + (size_t)bidx * p.bsc : nullptr;
  bf16_t* Cbp = p.Cb ? p.Cb + (size_t)bidx * p.bscb : nullptr;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < MN;
       e += (int64_t)gridDim.x * blockDim.x) {
    // eight partials in flight at a time, added in split order
    float s = 0.0f;
    for (int sp0 = 0; sp0 < p.splits; sp0 += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = (sp0 + u < p.splits) ? P[(size_t)(sp0 + u) * MN + e] : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    const int64_t row = e / p.N, col = e % p.N;
    float v = p.alpha * s;
    if (p.beta != 0.0f) v += p.beta * Cp[row * p.ldc + col];
    if (Cp) Cp[row * p.ldc + col] = v;
    if (Cbp) Cbp[row * p.ldcb + col] = f32_to_bf16(v);
  }
}

template <int MATH, int ADT, bool AKC, int BDT, bool BKC>
static void launch_t(hipStream_t s, dim3 g, const GemmParams& p) {
  hipLaunchKernelGGL((gemm_kernel<MATH, ADT, AKC, BDT, BKC>), g, dim3(GNT), 0, s, p);
}

template <int MATH, int ADT, bool AKC>
static void launch_b(hipStream_t s, dim3 g, const GemmParams& p, int bdt, bool bkc) {
  if (bdt == DT_F32) {
    if (bkc) launch_t<MATH, ADT, AKC, DT_F32, true>(s, g, p);
    else launch_t<MATH, ADT, AKC, DT_F32, false>(s, g, p);
  } else {
    if (bkc) launch_t<MATH, ADT, AKC, DT_BF16, true>(s, g, p);
    else launch_t<MATH, ADT, AKC, DT_BF16, false>(s, g, p);
  }
}

template <int MATH>
static void launch_a(hipStream_t s, dim3 g, const GemmParams& p, int adt, bool akc, int bdt,
                     bool bkc) {
  if (adt == DT_F32) {
    if (akc) launch_b<MATH, DT_F32, true>(s, g, p, bdt, bkc);
    else launch_b<MATH, DT_F32, false>(s, g, p, bdt, bkc);
  } else {
    if (akc) launch_b<MATH, DT_BF16, true>(s, g, p, bdt, bkc);
    else launch_b<MATH, DT_BF16, false>(s, g, p, bdt, bkc);
  }
}

static bool vec_ok(const MatRef& X) {
  const uintptr_t a = (uintptr_t)X.p;
  return (a % 16 == 0) && (X.ld % 8 == 0) && (X.bstride % 8 == 0);
}

// Stream-K plan of a plain product on the direct-to-LDS kernel (gemm_impl.h):
// lanes > 0 when it is estimated faster than the data-parallel grid (tile
// dp_mid, dp_splits split-K shares).  The estimates count slabs per
// workgroup in the slowest round: a 256-tile slab takes about 1.1 us (one
// workgroup per CU), a 128-tile slab 0.98 us with two workgroups on a CU and
// 0.75 us with one.  Split-K partials cost their fp32 traffic at 4 TB/s and
// a launch.  A stream-K walk pays for its share exchange, measured on
// MI355X at about 12 + 11 s us for 256 tiles and 10 + 4 s us for 128 tiles,
// s the number of lanes sharing a tile row: every lane's last share ends at
// the same moment, so the exchange is a burst at the end of the launch.
// Every lane count (a multiple of eight) up to the cap is tried.  So
// stream-K takes the long-K products with few output tiles (the Gram
// route's Gram columns: 1024 columns, K = p rows, whose 150-odd 256-tiles
// leave a second round of workgroups two-thirds empty), not the short-K ones.
// Stream-K is considered for K >= SK_MIN_K only.  Beside the factorisation's
// chain of small launches, short-K products did better data-parallel with
// split-K than stream-K (the Linear 4096 -> 11008 step, 13.06 against
// 13.20 ms with every plain product eligible): their workgroups are short-
// lived, so the chain finds CUs sooner, and their share exchange is a larger
// part of the launch.
constexpr int64_t SK_MIN_K = 8192;

struct SkPlan {
  int lanes = 0;
  bool mid = false;
  int iters = 0;
  size_t cnt_floats = 0;   // counter region (ints) at the head of the scratch
  size_t floats = 0;       // counters + partial tiles
};

static double slab_us(bool mid, int64_t wgs) {
  if (!mid) return 1.1;
  return wgs > 256 ? 0.98 : 0.75;
}

// lanes_max of the stream-K walk with tile `mid` (0 when not eligible)
static int64_t sk_lanes_max(int64_t M, int64_t N, int64_t K, bool mid, int max_wgs) {
  const int T = gemm_bb_tile(mid);
  const int64_t tn = cdiv(N, (int64_t)T), tm = cdiv(M, (int64_t)T);
  if (tn > 8) return 0;
  const int64_t U = tm * cdiv(K, (int64_t)gemm_bb_bk());
  int64_t G = mid ? 512 : 256;
  if (max_wgs > 0) G = std::min<int64_t>(G, max_wgs);
  int64_t L = std::min<int64_t>(G / tn, U / 8);
  return L - L % 8;
}

static size_t sk_floats(int64_t M, int64_t N, bool mid, int batch, int64_t L) {
  const int T = gemm_bb_tile(mid);
  const int64_t tn = cdiv(N, (int64_t)T), tm = cdiv(M, (int64_t)T);
  const size_t cntf = align_up((size_t)(batch * tm * tn), 64);
  return cntf + (size_t)batch * L * 2 * tn * T * T;
}

size_t gemm_scratch_floats(int64_t M, int64_t N, int64_t K, int batch, int max_wgs) {
  if (M < 1 || N < 1 || K < 1 || batch < 1) return 0;
  size_t f = 0;
  for (int c = 0; c < 2; ++c) {
    const int64_t L = sk_lanes_max(M, N, K, c == 1, max_wgs);
    if (L >= 8) f = std::max(f, sk_floats(M, N, c == 1, batch, L));
  }
  return f;
}

static SkPlan sk_choose(int64_t M, int64_t N, int64_t K, int batch, int max_wgs, bool dp_mid,
                        int dp_splits, size_t scratch_floats) {
  SkPlan best;
  const int bk = gemm_bb_bk();
  const int64_t I = cdiv(K, (int64_t)bk);
  // the data-parallel estimate
  double t_dp;
  {
    const int T = gemm_bb_tile(dp_mid);
    const int64_t wgs = cdiv(M, (int64_t)T) * cdiv(N, (int64_t)T) * dp_splits;
    int64_t G = dp_mid ? 512 : 256;
    if (max_wgs > 0) G = std::min<int64_t>(G, max_wgs);
    const int64_t rounds = cdiv(wgs, G);
    t_dp = (double)rounds * (double)cdiv(I, (int64_t)dp_splits) *
           slab_us(dp_mid, std::min<int64_t>(wgs, G));
    if (dp_splits > 1) t_dp += (double)dp_splits * (double)M * (double)N * 8.0 / 4.0e6 + 4.0;
  }
  double t_best = 0.9 * t_dp;   // stream-K only for a clear gain
  for (int c = 0; c < 2; ++c) {
    const bool mid = c == 1;
    const int T = gemm_bb_tile(mid);
    const int64_t tn = cdiv(N, (int64_t)T), tm = cdiv(M, (int64_t)T);
    const int64_t U = tm * I;
    for (int64_t L = sk_lanes_max(M, N, K, mid, max_wgs); L >= 8; L -= 8) {
      const size_t need = sk_floats(M, N, mid, batch, L);
      if (need > scratch_floats) continue;
      const int64_t s = cdiv(U, L);   // slabs per lane
      const double shares = s >= I ? 2.0 : (double)I / (double)s + 1.0;
      const double t = (double)s * slab_us(mid, L * tn) +
                       (mid ? 10.0 + 4.0 * shares : 12.0 + 11.0 * shares);
      if (t < t_best) {
        t_best = t;
        best.lanes = (int)L;
        best.mid = mid;
        best.iters = (int)I;
        best.cnt_floats = align_up((size_t)(batch * tm * tn), 64);
        best.floats = need;
      }
    }
  }
  return best;
}

int gemm(hipStream_t s, int math, int64_t M, int64_t N, int64_t K, float alpha, const MatRef& A,
         const MatRef& B, float beta, const OutRef& C, int batch, SplitScratch scratch,
         int max_wgs) {
  if (M < 0 || N < 0 || K < 0 || batch < 1) {
    set_error("gemm: negative size or batch < 1");
    return IFK_ERR_INVALID;
  }
  if (M == 0 || N == 0) return IFK_OK;
  if (!C.c && !C.cb) {
    set_error("gemm: no output");
    return IFK_ERR_INVALID;
  }
  if (beta != 0.0f && !C.c) {
    set_error("gemm: beta != 0 needs an fp32 output to read");
    return IFK_ERR_INVALID;
  }
  if (M > (int64_t)1 << 30 || N > (int64_t)1 << 30) {
    set_error("gemm: dimension too large");
    return IFK_ERR_INVALID;
  }
  GemmParams p;
  p.M = M; p.N = N; p.K = K; p.alpha = alpha; p.beta = beta;
  p.A = A.p; p.lda = A.ld; p.tria = A.tri; p.bsa = A.bstride;
  p.B = B.p; p.ldb = B.ld; p.trib = B.tri; p.bsb = B.bstride;
  p.C = C.c; p.ldc = C.ldc; p.bsc = C.bstride;
  p.Cb = C.cb; p.ldcb = C.ldcb; p.bscb = C.bstride_b;
  p.vec_a = vec_ok(A);
  p.vec_b = vec_ok(B);
  p.upper_only = C.upper && M == N;
  p.lower_only = C.lower && !C.upper;
  p.vec_c = (!C.c || ((uintptr_t)C.c % 16 == 0 && C.ldc % 4 == 0 && C.bstride % 4 == 0)) &&
            (!C.cb || ((uintptr_t)C.cb % 8 == 0 && C.ldcb % 4 == 0 && C.bstride_b % 4 == 0));
  // The 256 x 256 bf16 kernel takes the large contractions; small or fp32
  // ones stay on the 128 x 128 engine.
  const bool big = math == MATH_BF16 && M >= 192 && N >= 192 &&
                   (double)M * (double)N * (double)K * batch >= 1e9;
  // bf16 operands with K contiguous and 16-byte chunks: the direct-to-LDS
  // kernel, with its 256 tile when that alone gives most CUs a tile, else
  // with its 128 tile (four times the tiles, a quarter of the split-K
  // partials per tile)
  const bool bb = big && A.dt == DT_BF16 && A.kc && B.dt == DT_BF16 && B.kc && p.vec_a &&
                  p.vec_b && K % 8 == 0 && A.ld < ((int64_t)1 << 21) &&
                  B.ld < ((int64_t)1 << 21);
  // batch entries the tile and split-K choices are made for
  const int64_t bdec = C.per_entry ? 1 : batch;
  // split-K factor for a tile of TM x TN with BK-deep slabs
  auto split_for = [&](int TM, int TN, int BK, bool mid_tile) -> int {
    const int64_t tiles = cdiv(M, (int64_t)TM) * cdiv(N, (int64_t)TN) * bdec;
    const int64_t nkt = cdiv(K, (int64_t)BK);
    int64_t want = 1;
    if (mid_tile) {
      // one workgroup per CU, at least eight K slabs per split
      if (tiles < 256 && nkt >= 16) want = std::min<int64_t>(cdiv(256, tiles), nkt / 8);
    } else {
      // fewer tiles than this leave CUs idle (the direct-to-LDS kernel runs
      // one workgroup per CU, the others two); the direct-to-LDS kernel needs
      // a longer K per split to fill its ring
      const int64_t full = bb ? 224 : (big ? 160 : 192);
      if (tiles < full && nkt >= (bb ? 32 : 8))
        want = std::min<int64_t>(cdiv(2 * full, tiles), nkt / 4);
    }
    want = std::min<int64_t>(want, 64);
    while (want > 1 && (size_t)(want * batch) * (size_t)(M * N) > scratch.floats) --want;
    return (want > 1 && scratch.p) ? (int)want : 1;
  };
  // Direct-to-LDS tile: 256 when that alone gives most CUs a tile; else
  // whichever of 256 and 128 has the smaller estimated time -- the MFMA time
  // at the share of CUs its workgroups keep busy (the 128 tile runs at about
  // 0.55 of the 256 tile's rate per CU) plus its split-K partials (fp32,
  // written and read once).  Rates: 1.0e15 flop/s, 4e12 B/s.
  bool mid = false;
  if (bb) {
    const int T2 = gemm_bb_tile(false), T1 = gemm_bb_tile(true), bk = gemm_bb_bk();
    const int64_t t256 = cdiv(M, (int64_t)T2) * cdiv(N, (int64_t)T2) * bdec;
    if (t256 < 224) {
      const double fl = 2.0 * (double)M * (double)N * (double)K * bdec;
      auto est = [&](int T, bool mt, double rate) {
        const int sp = split_for(T, T, bk, mt);
        const double wgs = (double)(cdiv(M, (int64_t)T) * cdiv(N, (int64_t)T) * bdec) * sp;
        const double util = std::min(1.0, wgs / 256.0);
        const double part = sp > 1 ? (double)sp * (double)M * (double)N * bdec * 8.0 : 0.0;
        return fl / (1.0e15 * rate * util) + part / 4.0e12;
      };
      mid = est(T1, true, 0.55) < est(T2, false, 1.0);
    } else if ((A.tri != TRI_NONE || B.tri != TRI_NONE) && t256 < 300) {
      // a triangular operand gives tiles K ranges from 0 to K: with about one
      // round of 256 tiles the longest tile sets the time, and the 128 tile's
      // four times as many tiles, taken heaviest first, balance the CUs
      // (measured: 4096^3 with a triangular operand 160 -> 124 us; at 352
      // tiles of 256 the 256 tile stays ahead)
      mid = true;
    }
  }
  p.sk_lanes = 0;
  p.sk_iters = 0;
  p.sk_cnt = nullptr;
  p.sk_part = nullptr;
  if (bb && A.tri == TRI_NONE && B.tri == TRI_NONE && !p.upper_only &&
      !(p.lower_only && M == N) && K >= SK_MIN_K && scratch.p && (C.per_entry || batch == 1)) {
    const int T = gemm_bb_tile(mid);
    const int dp_splits = split_for(T, T, gemm_bb_bk(), mid);
    const SkPlan sk = sk_choose(M, N, K, batch, max_wgs, mid, dp_splits, scratch.floats);
    if (sk.lanes > 0) {
      mid = sk.mid;
      p.sk_lanes = sk.lanes;
      p.sk_iters = sk.iters;
      p.sk_cnt = reinterpret_cast<int*>(scratch.p);
      p.sk_part = scratch.p + sk.cnt_floats;
    }
  }
  const int TM = bb ? gemm_bb_tile(mid) : (big ? gemm_big_tile_m() : GBM);
  const int TN = bb ? gemm_bb_tile(mid) : (big ? gemm_big_tile_n() : GBN);
  p.tiles_m = (int)cdiv(M, TM);
  p.tiles_n = (int)cdiv(N, TN);
  const int BK = bb ? gemm_bb_bk()
                    : big ? gemm_big_bk()
                          : (math == MATH_BF16 ? GCfg<MATH_BF16>::BK : GCfg<MATH_F32>::BK);
  const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n * batch;
  const int splits = p.sk_lanes > 0 ? 1 : split_for(TM, TN, BK, mid);
  p.splits = splits;
  p.part = splits > 1 ? scratch.p : nullptr;
  if (tiles * splits > 0x7fffffffLL || (int64_t)batch * splits > 65535) {
    set_error("gemm: grid too large");
    return IFK_ERR_INVALID;
  }
  unsigned gx = (unsigned)(p.tiles_m * p.tiles_n);
  // a square output of which one triangle is wanted: the direct-to-LDS
  // kernel enumerates the live tiles only
  if (bb && (p.upper_only || p.lower_only) && M == N && p.tiles_m == p.tiles_n)
    gx = (unsigned)(p.tiles_m * (p.tiles_m + 1) / 2);
  if (big && max_wgs > 0) {
    const int64_t per_z = std::max<int64_t>(1, max_wgs / std::max<int64_t>(1, batch * splits));
    gx = (unsigned)std::min<int64_t>(gx, per_z);
  }
  // the direct-to-LDS kernel orders its tiles by XCD when a z slice has a
  // multiple of eight workgroups (the rest of the tiles go grid-stride)
  if (bb && gx > 8) gx &= ~7u;
  // stream-K: one workgroup per lane and tile column (the lanes were chosen
  // for one entry within the cap), the arrival counters zeroed first
  if (p.sk_lanes > 0) {
    gx = (unsigned)(p.sk_lanes * p.tiles_n);
    const int rc0 = launch_fill_int(s, p.sk_cnt, 0, (int)(batch * p.tiles_m * p.tiles_n));
    if (rc0) return rc0;
  }
  dim3 grid(gx, 1, (unsigned)(batch * splits));
  const int vid = gemm_variant_id(math, A.dt, A.kc, B.dt, B.kc) | ((big ? 1 : 0) << 5) |
                  ((bb ? 1 : 0) << 6) | ((mid ? 1 : 0) << 7) |
                  ((p.sk_lanes > 0 ? 1 : 0) << 9);
  ProfRec* pr = prof_slot(vid);
  if (pr) {
    // algorithmic work: 2 K times the wanted outputs (M N, or one triangle of
    // them), halved when one operand is triangular; and the minimal traffic:
    // each operand read once, C read (beta != 0) and written once
    const double tri = (A.tri != TRI_NONE || B.tri != TRI_NONE) ? 0.5 : 1.0;
    double live = (double)M * (double)N;
    if (p.upper_only) live = (double)N * (double)(N + 1) / 2.0;
    else if (p.lower_only)
      live = M >= N ? (double)M * (double)N - (double)N * (double)(N - 1) / 2.0
                    : (double)M * (double)(M + 1) / 2.0;
    pr->variant = vid;
    pr->m = M;
    pr->n = N;
    pr->k = K;
    pr->flops = 2.0 * tri * live * (double)K * batch;
    const double sa = A.dt == DT_F32 ? 4 : 2, sb = B.dt == DT_F32 ? 4 : 2;
    double cb = (C.c ? 4.0 : 0.0) + (C.cb ? 2.0 : 0.0) + (beta != 0.0f ? 4.0 : 0.0);
    pr->bytes = ((double)M * K * sa + (double)K * N * sb + (double)M * N * cb) * batch;
    hipEventRecord(pr->beg, s);
  }
  if (bb) launch_gemm_bb(s, grid, p, mid);
  else if (big) launch_gemm_big(s, grid, p, A.dt, A.kc, B.dt, B.kc);
  else if (math == MATH_BF16) launch_a<MATH_BF16>(s, grid, p, A.dt, A.kc, B.dt, B.kc);
  else launch_a<MATH_F32>(s, grid, p, A.dt, A.kc, B.dt, B.kc);
  if (pr) hipEventRecord(pr->end, s);
  int rc = check_launch("gemm");
  if (rc) return rc;
  if (splits > 1) {
    int64_t MN = M * N;
    unsigned gx = (unsigned)std::min<int64_t>(cdiv(MN, 256), 4096);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(gx, batch), dim3(256), 0, s, p);
    rc = check_launch("gemm splitk reduce");
  }
  return rc;
}

}  // namespace ifk
