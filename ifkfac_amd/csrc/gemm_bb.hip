// bf16 x bf16 GEMM for operands whose K index is contiguous in memory:
//   C = alpha * A B^T + beta * C,  A[m][k] (lda), B[n][k] (ldb), fp32 accumulation,
// fp32 C and/or an RNE bf16 copy, batched and split-K like the rest of the
// engine (gemm.h).  This is the kernel of the fold's outer-block updates and
// of the preconditioner's products.
//
// Two tiles share the code.  The large one, 256 x 256 x 32 with eight waves
// of 128 x 64 (4 x 2 v_mfma_f32_32x32x16_bf16 tiles each, 128 fp32
// accumulators per lane) and one workgroup per CU, takes products with many
// output tiles: the square tile halves the operand bytes per flop of a
// 256 x 128 tile, which matters because the kernel is bound by how fast
// slabs reach LDS, not by LDS bandwidth (no bank conflicts, LDS about 10 %
// busy).  The mid one, 128 x 128 x 32 with four waves of 64 x 64 and two
// workgroups per CU, takes products with few output rows or columns (the
// fold's 512-wide outer-block products): four times the tiles fill the CUs
// without split-K, or with a quarter of the split-K partial traffic.
// Operand slabs go from global memory straight into LDS
// (buffer_load_dwordx4 ... lds), so staging costs no registers and the
// workgroup keeps a ring of four slabs (128 / 64 KB): the loads of slabs
// k + 1 .. k + 3 are in flight while slab k is multiplied.  Buffer
// descriptors bound each operand, so rows past M / N read as zero without a
// branch.  The 64-byte rows of a slab are stored with their four 16-byte
// chunks XOR-swizzled by bits 2-3 of the row, which makes the MFMA fragment
// reads (ds_read_b128 of 16 rows x one chunk) bank-conflict free.
//
// Requirements checked by the dispatcher: K, lda, ldb multiples of 8 and
// 16-byte aligned operand pointers (a 16-byte chunk never straddles K).
// Triangular operands: the K range of a tile is trimmed to the structurally
// non-zero part, and slabs that cross the diagonal are masked after the
// fragment reads.
#include "common.h"
#include "gemm_impl.h"

namespace ifk {

namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int BK = 32, STAGES = 4;

template <int BM_, int BN_, int WAVES_M_, int WAVES_N_, int OCC_, bool PIPE_ = false>
struct BbCfg {
  static constexpr int BM = BM_, BN = BN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_, OCC = OCC_;
  static constexpr bool PIPE = PIPE_;   // fragment reads one half-slab ahead (see bb_tile)
  static constexpr int NWAVE = WAVES_M * WAVES_N, NTH = NWAVE * 64;
  static constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;   // wave tile
  static constexpr int FM = WTM / 32, FN = WTN / 32;             // 32 x 32 MFMA tiles per wave
  static constexpr int SLAB_A = BM * BK, SLAB_B = BN * BK;       // bf16 elements per slab
  static constexpr int STAGE = SLAB_A + SLAB_B;
  static constexpr int LOADS_A = SLAB_A * 2 / 16 / NTH;          // 16-byte loads per thread
  static constexpr int LOADS_B = SLAB_B * 2 / 16 / NTH;
  static constexpr int LOADS = LOADS_A + LOADS_B;                // per thread per slab pair
  static_assert(2 * LOADS <= 63, "vmcnt holds at most 63 loads in flight");
  static_assert(SLAB_A * 2 % (16 * NTH) == 0 && SLAB_B * 2 % (16 * NTH) == 0, "slab split");
};
using BigCfg = BbCfg<256, 256, 2, 4, 1, true>;   // 512 threads, 128 KB ring, one WG per CU
using MidCfg = BbCfg<128, 128, 2, 2, 2>;   // 256 threads, 64 KB ring, two workgroups per CU

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int nrec = bytes > 0x7ffffff0LL ? 0x7ffffff0 : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, nrec, 0x00020000);
}

// Per-thread addressing of the slab loads, fixed for a tile: wave w,
// instruction i fills slots (NWAVE i + w) * 64 .. + 63; lane l's slot
// s = (row, q) holds the logical chunk c = q ^ ((row >> 2) & 3) of that row,
// i.e. byte offset row * ld * 2 + 16 c of the operand view plus 64 per K
// slab (row < 256 and ld < 2^21 keep it in 32 bits), and K index 8 c plus
// 32 per slab.
template <int NWAVE, int NL>
struct SlabAddr {
  unsigned base[NL];
  int kc[NL];
  __device__ __forceinline__ void init(int64_t ld) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int slot = (i * NWAVE + wave) * 64 + lane;
      const int row = slot >> 2, q = slot & 3;
      const int c = q ^ ((row >> 2) & 3);
      base[i] = (unsigned)((int64_t)row * ld * 2) + 16u * (unsigned)c;
      kc[i] = 8 * c;
    }
  }
};

// Issue the loads of one operand slab (K chunk kt) into LDS S.  Chunks at or
// past K read as zero (the offset is beyond the buffer).
template <int NWAVE, int NL>
__device__ __forceinline__ void issue_slab(__amdgpu_buffer_rsrc_t rs, bf16_t* S,
                                           const SlabAddr<NWAVE, NL>& a, int kt, int kmax) {
  // the LDS destination (M0) must be wave-uniform: take the wave index from
  // a scalar register so the compiler knows it
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int k0 = kt * BK;
  const unsigned koff = (unsigned)k0 * 2u;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int slot0 = (i * NWAVE + wave) * 64;
    const unsigned off = (k0 + a.kc[i] < kmax) ? a.base[i] + koff : 0x80000000u;
    lds_void* dst = (lds_void*)(uintptr_t)(S + slot0 * 8);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, off, 0, 0, 0);
  }
}

__device__ __forceinline__ bf16x8_t frag(const bf16_t* S, int row, int c) {
  return *(const bf16x8_t*)(S + row * BK + ((c ^ ((row >> 2) & 3)) << 3));
}

// Zero the entries of an 8-element fragment (row index mn, k = k0 .. k0 + 7)
// that lie in the structurally zero triangle: op(X)[mn][k] for A-side (ISA)
// or op(X)[k][mn] for B-side operands.
template <bool ISA>
__device__ __forceinline__ bf16x8_t mask_frag(bf16x8_t v, int tri, int64_t mn, int64_t k0) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t k = k0 + e;
    bool zero;
    if (ISA) zero = (tri == TRI_UPPER) ? (k < mn) : (k > mn);
    else zero = (tri == TRI_UPPER) ? (k > mn) : (k < mn);
    if (zero) v[e] = (__bf16)0.0f;
  }
  return v;
}

// Whether the diagonal k == mn passes through the slab [mn0, mn0 + ext) x
// [k0, k0 + 32) of a triangular operand (else the slab is all structural
// non-zeros: the K range of the tile already excludes the all-zero slabs).
__device__ __forceinline__ bool slab_crosses(int tri, int64_t mn0, int ext, int64_t k0) {
  if (tri == TRI_NONE) return false;
  return k0 < mn0 + ext && k0 + BK > mn0;
}

// s_waitcnt immediate for vmcnt(n) with expcnt and lgkmcnt left alone
// (vmcnt bits 3:0 and 15:14, expcnt 6:4 = 7, lgkmcnt 11:8 = 15)
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0f70; }

// Wait until the loads of this slab have landed, leaving those of the
// `ahead` later slabs already issued (0, 1 or 2: L loads each) in flight.
template <int L>
__device__ __forceinline__ void wait_vm(int ahead) {
  if (ahead >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * L));
  else if (ahead == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(L));
  else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
}

// The fragments of one K half (16) of a slab: FM rows of A, FN rows of B,
// masked where a triangular operand's slab crosses the diagonal.
template <class CF, bool TRI>
struct Frags {
  bf16x8_t a[CF::FM], b[CF::FN];
  __device__ __forceinline__ void read(const bf16_t* As, const bf16_t* Bs, int ks, int wm, int wn,
                                       int l32, int h) {
#pragma unroll
    for (int i = 0; i < CF::FM; ++i) a[i] = frag(As, wm * CF::WTM + i * 32 + l32, 2 * ks + h);
#pragma unroll
    for (int j = 0; j < CF::FN; ++j) b[j] = frag(Bs, wn * CF::WTN + j * 32 + l32, 2 * ks + h);
  }
  __device__ __forceinline__ void mask(const GemmParams& p, int64_t m0, int64_t n0, int64_t kbase,
                                       int ks, int wm, int wn, int l32, int h) {
    if (!TRI) return;
    if (slab_crosses(p.tria, m0, CF::BM, kbase)) {
#pragma unroll
      for (int i = 0; i < CF::FM; ++i)
        a[i] = mask_frag<true>(a[i], p.tria, m0 + wm * CF::WTM + i * 32 + l32,
                               kbase + ks * 16 + h * 8);
    }
    if (slab_crosses(p.trib, n0, CF::BN, kbase)) {
#pragma unroll
      for (int j = 0; j < CF::FN; ++j)
        b[j] = mask_frag<false>(b[j], p.trib, n0 + wn * CF::WTN + j * 32 + l32,
                                kbase + ks * 16 + h * 8);
    }
  }
};

template <class CF>
__device__ __forceinline__ void mfma_all(f32x16_t (&acc)[CF::FM][CF::FN], const bf16x8_t* a,
                                         const bf16x8_t* b) {
#pragma unroll
  for (int i = 0; i < CF::FM; ++i)
#pragma unroll
    for (int j = 0; j < CF::FN; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
}

// Main loop with the fragment reads one K half ahead of the products that
// use them, for configurations of one wave per SIMD (no second wave to cover
// the LDS latency).  Per slab: read the second half's fragments, multiply
// the first half's, then wait for the next slab's loads and meet at the
// barrier (after it every wave is past its reads of the previous slab, whose
// ring slot then takes the slab STAGES - 1 ahead), read the next slab's first
// half, multiply this slab's second half.  So the barrier and the LDS
// latency fall under a half slab of products.
template <class CF, bool TRI>
__device__ __forceinline__ void pipe_loop(const GemmParams& p, f32x16_t (&acc)[CF::FM][CF::FN],
                                          bf16_t* smem, __amdgpu_buffer_rsrc_t ra,
                                          __amdgpu_buffer_rsrc_t rb,
                                          const SlabAddr<CF::NWAVE, CF::LOADS_A>& aa,
                                          const SlabAddr<CF::NWAVE, CF::LOADS_B>& ab, int kmax,
                                          int64_t kt0, int n_it, int64_t m0, int64_t n0, int wm,
                                          int wn, int l32, int h) {
  constexpr int STAGE = CF::STAGE, SLAB_A = CF::SLAB_A;
  if (n_it <= 0) return;
  // prologue: slabs 0 .. STAGES - 2 in flight, slab 0 landed everywhere
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) {
    if (s < n_it) {
      issue_slab(ra, smem + s * STAGE, aa, (int)(kt0 + s), kmax);
      issue_slab(rb, smem + s * STAGE + SLAB_A, ab, (int)(kt0 + s), kmax);
    }
  }
  wait_vm<CF::LOADS>(min(n_it - 1, STAGES - 2));
  __builtin_amdgcn_s_barrier();
  Frags<CF, TRI> f0, f1;
  f0.read(smem, smem + SLAB_A, 0, wm, wn, l32, h);
  f0.mask(p, m0, n0, kt0 * BK, 0, wm, wn, l32, h);
  for (int it = 0; it < n_it; ++it) {
    const bf16_t* As = smem + (it % STAGES) * STAGE;
    const int64_t kbase = (kt0 + it) * BK;
    f1.read(As, As + SLAB_A, 1, wm, wn, l32, h);
    f1.mask(p, m0, n0, kbase, 1, wm, wn, l32, h);
    mfma_all<CF>(acc, f0.a, f0.b);
    if (it + 1 < n_it) {
      // slab it + 1 landed (the slabs issued after it may fly), every wave
      // past its reads of slab it - 1
      wait_vm<CF::LOADS>(min(STAGES - 3, n_it - 2 - it));
      __builtin_amdgcn_s_barrier();
      if (it + STAGES - 1 < n_it) {
        const int sn = (it + STAGES - 1) % STAGES;
        issue_slab(ra, smem + sn * STAGE, aa, (int)(kt0 + it + STAGES - 1), kmax);
        issue_slab(rb, smem + sn * STAGE + SLAB_A, ab, (int)(kt0 + it + STAGES - 1), kmax);
      }
      const bf16_t* An = smem + ((it + 1) % STAGES) * STAGE;
      f0.read(An, An + SLAB_A, 0, wm, wn, l32, h);
      f0.mask(p, m0, n0, kbase + BK, 0, wm, wn, l32, h);
    }
    mfma_all<CF>(acc, f1.a, f1.b);
  }
}

// Products of tile (m0, n0) of entry bidx over K slabs [kt0, kt0 + n_it):
// acc = A_tile B_tile^T (zero when n_it <= 0).  TRI: a triangular operand
// (slabs across the diagonal masked).
template <class CF, bool TRI>
__device__ __forceinline__ void bb_acc(const GemmParams& p, int bidx, int64_t m0, int64_t n0,
                                       int64_t kt0, int n_it, f32x16_t (&acc)[CF::FM][CF::FN],
                                       bf16_t* smem) {
  constexpr int BM = CF::BM, BN = CF::BN, FM = CF::FM, FN = CF::FN;
  constexpr int STAGE = CF::STAGE, SLAB_A = CF::SLAB_A;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave / CF::WAVES_N, wn = wave % CF::WAVES_N;
  const int l32 = lane & 31, h = lane >> 5;

  const bf16_t* Ab = (const bf16_t*)p.A + (size_t)bidx * p.bsa + m0 * p.lda;
  const bf16_t* Bb = (const bf16_t*)p.B + (size_t)bidx * p.bsb + n0 * p.ldb;
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(Ab, (p.M - m0) * p.lda * 2);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(Bb, (p.N - n0) * p.ldb * 2);
  SlabAddr<CF::NWAVE, CF::LOADS_A> aa;
  SlabAddr<CF::NWAVE, CF::LOADS_B> ab;
  aa.init(p.lda);
  ab.init(p.ldb);
  const int kmax = (int)p.K;

#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  if constexpr (CF::PIPE) {
    pipe_loop<CF, TRI>(p, acc, smem, ra, rb, aa, ab, kmax, kt0, n_it, m0, n0, wm, wn, l32, h);
  } else {
    // prologue: slabs 0 .. STAGES - 2
  #pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) {
      if (s < n_it) {
        issue_slab(ra, smem + s * STAGE, aa, (int)(kt0 + s), kmax);
        issue_slab(rb, smem + s * STAGE + SLAB_A, ab, (int)(kt0 + s), kmax);
      }
    }
    for (int it = 0; it < n_it; ++it) {
      wait_vm<CF::LOADS>(min(n_it - 1 - it, STAGES - 2));   // this slab landed (later ones may fly)
      // every wave's loads of this slab are in LDS and slab it - 1 is free
      // again.  A bare s_barrier: __syncthreads() would also wait for the next
      // slab's loads (its fence drains vmcnt).
      __builtin_amdgcn_s_barrier();
      if (it + STAGES - 1 < n_it) {
        const int sn = (it + STAGES - 1) % STAGES;
        issue_slab(ra, smem + sn * STAGE, aa, (int)(kt0 + it + STAGES - 1), kmax);
        issue_slab(rb, smem + sn * STAGE + SLAB_A, ab, (int)(kt0 + it + STAGES - 1), kmax);
      }
      const bf16_t* As = smem + (it % STAGES) * STAGE;
      const bf16_t* Bs = As + SLAB_A;
      const int64_t kbase = (kt0 + it) * BK;
      const bool xa = TRI && slab_crosses(p.tria, m0, BM, kbase);
      const bool xb = TRI && slab_crosses(p.trib, n0, BN, kbase);
  #pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        bf16x8_t af[FM], bfr[FN];
  #pragma unroll
        for (int i = 0; i < FM; ++i) af[i] = frag(As, wm * CF::WTM + i * 32 + l32, 2 * ks + h);
  #pragma unroll
        for (int j = 0; j < FN; ++j) bfr[j] = frag(Bs, wn * CF::WTN + j * 32 + l32, 2 * ks + h);
        if (xa) {
  #pragma unroll
          for (int i = 0; i < FM; ++i)
            af[i] = mask_frag<true>(af[i], p.tria, m0 + wm * CF::WTM + i * 32 + l32,
                                    kbase + ks * 16 + h * 8);
        }
        if (xb) {
  #pragma unroll
          for (int j = 0; j < FN; ++j)
            bfr[j] = mask_frag<false>(bfr[j], p.trib, n0 + wn * CF::WTN + j * 32 + l32,
                                      kbase + ks * 16 + h * 8);
        }
  #pragma unroll
        for (int i = 0; i < FM; ++i)
  #pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      }
    }
  }
}

// Tile (m0, n0) of entry bidx: C = alpha acc + beta C, and the bf16 copy.
// acc[i][j][r] holds row (r / 4) * 8 + h * 4 + r % 4, column l32 of 32 x 32
// tile (i, j) of the wave.  Uses the LDS ring (every wave must be past its
// last fragment reads; the first barrier below sees to that).
template <class CF>
__device__ __forceinline__ void bb_store(const GemmParams& p, int bidx, int64_t m0, int64_t n0,
                                         const f32x16_t (&acc)[CF::FM][CF::FN], bf16_t* smem) {
  constexpr int BN = CF::BN, FM = CF::FM, FN = CF::FN;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave / CF::WAVES_N, wn = wave % CF::WAVES_N;
  const int l32 = lane & 31, h = lane >> 5;
  float* Cp = p.C ? p.C + (size_t)bidx * p.bsc : nullptr;
  bf16_t* Cbp = p.Cb ? p.Cb + (size_t)bidx * p.bscb : nullptr;
  if (p.vec_c) {
    // Through LDS, one 32-row band of each wave row at a time: the band is
    // read back row-contiguous, so C is read and written 16 bytes and the bf16
    // copy 8 bytes per lane.
    constexpr int LDB = BN + 4;                        // band row stride (floats)
    constexpr int V4 = BN / 4;                         // float4 per band row
    static_assert(CF::WAVES_M * 32 * LDB * 4 <= STAGES * CF::STAGE * 2, "band fits the ring");
    float* band = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      __syncthreads();
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          band[(wm * 32 + (r >> 2) * 8 + h * 4 + (r & 3)) * LDB + wn * CF::WTN + j * 32 + l32] =
              acc[i][j][r];
      __syncthreads();
      for (int idx = t; idx < CF::WAVES_M * 32 * V4; idx += CF::NTH) {
        const int rb = idx / V4, c4 = idx - rb * V4;
        const int64_t row = m0 + (rb >> 5) * CF::WTM + i * 32 + (rb & 31);
        const int64_t col = n0 + c4 * 4;
        if (row >= p.M || col >= p.N) continue;
        const float4 a = *reinterpret_cast<const float4*>(band + rb * LDB + c4 * 4);
        float v[4] = {p.alpha * a.x, p.alpha * a.y, p.alpha * a.z, p.alpha * a.w};
        if (col + 3 < p.N) {
          if (p.beta != 0.0f) {
            const float4 o = *reinterpret_cast<const float4*>(Cp + row * p.ldc + col);
            v[0] += p.beta * o.x; v[1] += p.beta * o.y; v[2] += p.beta * o.z; v[3] += p.beta * o.w;
          }
          if (Cp) *reinterpret_cast<float4*>(Cp + row * p.ldc + col) = make_float4(v[0], v[1], v[2], v[3]);
          if (Cbp) {
            const unsigned lo = (unsigned)f32_to_bf16(v[0]) | ((unsigned)f32_to_bf16(v[1]) << 16);
            const unsigned hi = (unsigned)f32_to_bf16(v[2]) | ((unsigned)f32_to_bf16(v[3]) << 16);
            *reinterpret_cast<uint2*>(Cbp + row * p.ldcb + col) = make_uint2(lo, hi);
          }
        } else {
          for (int u = 0; u < 4 && col + u < p.N; ++u) {
            float x = v[u];
            if (p.beta != 0.0f) x += p.beta * Cp[row * p.ldc + col + u];
            if (Cp) Cp[row * p.ldc + col + u] = x;
            if (Cbp) Cbp[row * p.ldcb + col + u] = f32_to_bf16(x);
          }
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t col = n0 + wn * CF::WTN + j * 32 + l32;
      float old[16];
      if (p.beta != 0.0f) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * CF::WTM + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
          old[r] = (row < p.M && col < p.N) ? Cp[row * p.ldc + col] : 0.0f;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * CF::WTM + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
        if (row < p.M && col < p.N) {
          float v = p.alpha * acc[i][j][r];
          if (p.beta != 0.0f) v += p.beta * old[r];
          if (Cp) Cp[row * p.ldc + col] = v;
          if (Cbp) Cbp[row * p.ldcb + col] = f32_to_bf16(v);
        }
      }
    }
}

// One output tile, or one split-K share of it (grid.z = batch * splits).
// TRI: a triangular operand (K range trimmed to the structural non-zeros).
template <class CF, bool TRI>
__device__ __forceinline__ void bb_tile(const GemmParams& p, int tm, int tn, bf16_t* smem) {
  constexpr int BM = CF::BM, BN = CF::BN, FM = CF::FM, FN = CF::FN;
  const int z = blockIdx.z;
  const int bidx = z / p.splits, split = z % p.splits;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  if (p.upper_only && m0 >= n0 + BN) return;   // wholly below the diagonal
  if (p.lower_only && n0 >= m0 + BM) return;   // wholly above the diagonal

  int64_t klo = 0, khi = p.K;
  if (p.tria == TRI_UPPER) klo = max(klo, m0);
  if (p.tria == TRI_LOWER) khi = min(khi, m0 + BM);
  if (p.trib == TRI_UPPER) khi = min(khi, n0 + BN);
  if (p.trib == TRI_LOWER) klo = max(klo, n0);
  const int64_t kt_lo = klo / BK;
  const int64_t nkt = khi > kt_lo * BK ? (khi - kt_lo * BK + BK - 1) / BK : 0;
  const int64_t per = (nkt + p.splits - 1) / p.splits;
  const int64_t kt0 = kt_lo + (int64_t)split * per;
  const int64_t kt1 = min(kt_lo + nkt, kt0 + per);
  const int n_it = (int)max((int64_t)0, kt1 - kt0);

  f32x16_t acc[FM][FN];
  bb_acc<CF, TRI>(p, bidx, m0, n0, kt0, n_it, acc, smem);

  if (p.splits > 1) {
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int wm = wave / CF::WAVES_N, wn = wave % CF::WAVES_N;
    const int l32 = lane & 31, h = lane >> 5;
    float* P = p.part + ((size_t)(bidx * p.splits + split)) * (size_t)p.M * (size_t)p.N;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * CF::WTM + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
          const int64_t col = n0 + wn * CF::WTN + j * 32 + l32;
          if (row < p.M && col < p.N) P[row * p.N + col] = acc[i][j][r];
        }
    return;
  }
  bb_store<CF>(p, bidx, m0, n0, acc, smem);
}

// Partial tile slot of a stream-K lane: slot `which` (0: the first tile row
// the lane touches, 1: its last) of tile column col, entry bidx.  A slot holds
// the workgroup's accumulators in register order, 16 bytes per thread.
template <class CF>
__device__ __forceinline__ float* sk_slot(const GemmParams& p, int bidx, int lane, int which,
                                          int col) {
  const size_t idx = (((size_t)bidx * p.sk_lanes + lane) * 2 + which) * p.tiles_n + col;
  return p.sk_part + idx * (size_t)(CF::BM * CF::BN);
}

// A partial tile's buffer descriptor.  The shares move between workgroups
// (on any XCD, each with its own L2) by device-scope stores and loads
// (cache policy SC1, what relaxed agent-scope atomic stores and loads of the
// memory model use): coherent without the L2 write-back and invalidation of
// a device-scope fence.
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
constexpr int CPOL_SC1 = 16;
template <class CF>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slot_rsrc(float* S) {
  return make_rsrc(S, (int64_t)CF::BM * CF::BN * 4);
}

// Stream-K walk of one workgroup (lane, tile column col): tile rows
// u0 / I .. (u1 - 1) / I of its share [u0, u1) of the U = tiles_m * I
// (row, slab) steps.  A tile whose K range lies wholly in the share is
// stored directly.  Otherwise every lane that holds part of it stores its
// partial tile by device-scope stores, waits for them to complete, and counts
// itself in on the tile's counter (a device-scope atomic); the one that
// arrives last reads the partials by device-scope loads, adds them in lane
// order and stores the tile.  (The first lane of a row, which usually
// arrives last, first looks at the counter and skips its own store when the
// others are all in.)  Nobody waits for anybody, so the walk ends
// whatever order the workgroups run in, and the sum's order does not depend
// on the arrival order: the result is deterministic.
template <class CF>
__device__ __forceinline__ void bb_streamk(const GemmParams& p, bf16_t* smem, int* s_old) {
  constexpr int BM = CF::BM, BN = CF::BN, FM = CF::FM, FN = CF::FN, NTH = CF::NTH;
  const int tn_ = p.tiles_n, L = p.sk_lanes, I = p.sk_iters;
  const int bidx = blockIdx.z;
  // workgroup x runs on XCD x % 8: the lanes of one XCD take consecutive
  // shares, so most shared tiles are summed within one L2
  const int per_xcd = (int)(gridDim.x >> 3);
  const int pos = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  const int lane = pos / tn_, col = pos - lane * tn_;
  const int64_t U = (int64_t)p.tiles_m * I;
  const int64_t u0 = (int64_t)lane * U / L, u1 = (int64_t)(lane + 1) * U / L;
  const int64_t r_first = u0 / I;
  const int t = threadIdx.x;
  for (int64_t r = r_first; r * I < u1; ++r) {
    const int64_t s0 = max(u0, r * I) - r * I, s1 = min(u1, (r + 1) * I) - r * I;
    const int64_t m0 = r * BM, n0 = (int64_t)col * BN;
    if (p.upper_only && m0 >= n0 + BN) continue;   // every lane skips the same tiles
    if (p.lower_only && n0 >= m0 + BM) continue;
    f32x16_t acc[FM][FN];
    bb_acc<CF, false>(p, bidx, m0, n0, s0, (int)(s1 - s0), acc, smem);
    // a tile wholly in this share is stored directly; a shared one by the
    // last lane to arrive
    bool store = true;
    if (!(s0 == 0 && s1 == I)) {
      const int lf = sk_lane_of(r * I, U, L), ll = sk_lane_of((r + 1) * I - 1, U, L);
      int* cnt = p.sk_cnt + ((int64_t)bidx * p.tiles_m + r) * tn_ + col;
      // The row's first lane usually arrives last: its share of the row ends
      // its walk, the other lanes' shares begin (or make up) theirs.  When a
      // look at the counter shows every other share in, it adds them to its
      // own accumulators, which hold the first term of the sum, and stores
      // nothing of its own.
      int seen = -1;
      if (lane == lf) {
        if (t == 0) *s_old = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        seen = *s_old;
        __syncthreads();
      }
      int first_mem = lf + 1;   // the first share read from memory
      if (seen != ll - lf) {
        first_mem = lf;
        const __amdgpu_buffer_rsrc_t rs =
            slot_rsrc<CF>(sk_slot<CF>(p, bidx, lane, r == r_first ? 0 : 1, col));
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              u32x4_t v;
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = __float_as_uint(acc[i][j][4 * q + e]);
              __builtin_amdgcn_raw_buffer_store_b128(
                  v, rs, (unsigned)((((i * FN + j) * 4 + q) * NTH + t) * 16), 0, CPOL_SC1);
            }
        // the device-scope stores have completed (so every other lane sees
        // them) before the count
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();
        if (t == 0) *s_old = atomicAdd(cnt, 1);
        __syncthreads();
        store = *s_old == ll - lf;
      }
      if (store) {
        // the shares in lane order by device-scope loads (the first lane's
        // from its registers when it never stored it), summed into the
        // accumulators: the same additions in the same order either way
        for (int l = first_mem; l <= ll; ++l) {
          const int wh = (r == ((int64_t)l * U / L) / I) ? 0 : 1;
          const __amdgpu_buffer_rsrc_t rs = slot_rsrc<CF>(sk_slot<CF>(p, bidx, l, wh, col));
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(
                    rs, (unsigned)((((i * FN + j) * 4 + q) * NTH + t) * 16), 0, CPOL_SC1);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  if (l == lf) acc[i][j][4 * q + e] = __uint_as_float(x[e]);
                  else acc[i][j][4 * q + e] += __uint_as_float(x[e]);
                }
              }
        }
      }
    }
    if (store) bb_store<CF>(p, bidx, m0, n0, acc, smem);
    __syncthreads();   // the ring and *s_old are reused by the next tile
  }
}

// Tile order.  Workgroups go to the eight XCDs round-robin by their linear
// id, and each XCD has its own L2, so with a multiple of eight workgroups per
// z slice (workgroup x runs on XCD x % 8) XCD c takes the c-th eighth of the
// tiles in grouped order -- bands of XCD_GM tile rows, walked down the band
// first -- and its workgroups step through that range together: the tiles
// in flight on one XCD share a few row and column operand strips, which stay
// in its L2 instead of being fetched again for every tile.  Other grids, and
// products with a triangular operand (whose tiles differ in K range, so
// contiguous ranges would load some XCDs more than others), visit tiles
// grid-stride, heaviest first (tile_order).  A square output of which only
// one triangle is wanted enumerates the live tiles only (row by row of the
// wanted triangle), so that the skipped ones do not leave some XCDs idle.
constexpr int XCD_GM = 8;

// Live tile l (0 .. T (T + 1) / 2 - 1) of a T x T tile grid of which only the
// lower triangle (upper = false) or the upper one is wanted: row r of the
// triangle holds tiles (r, 0 .. r).
__device__ __forceinline__ void tri_tile(int l, bool upper, int* tm, int* tn) {
  int r = (int)((sqrtf(8.0f * (float)l + 1.0f) - 1.0f) * 0.5f);
  while (r > 0 && r * (r + 1) / 2 > l) --r;
  while ((r + 1) * (r + 2) / 2 <= l) ++r;
  const int c = l - r * (r + 1) / 2;
  *tm = upper ? c : r;
  *tn = upper ? r : c;
}

template <class CF>
__global__ __launch_bounds__(CF::NTH, CF::OCC) void gemm_bb_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) bf16_t smem_bb[STAGES * CF::STAGE];
  __shared__ int s_old;
  const int tiles_m = p.tiles_m, tiles_n = p.tiles_n;
  const int tiles = tiles_m * tiles_n;
  if (p.sk_lanes > 0) {
    bb_streamk<CF>(p, smem_bb, &s_old);
  } else if ((p.upper_only || p.lower_only) && tiles_m == tiles_n && p.M == p.N) {
    const int live = tiles_m * (tiles_m + 1) / 2;
    const bool xcd = (gridDim.x & 7) == 0;
    const int c = xcd ? (int)(blockIdx.x & 7) : 0, nl = xcd ? (int)(gridDim.x >> 3) : gridDim.x;
    const int per = xcd ? (live + 7) >> 3 : live;
    const int l1 = min(live, (c + 1) * per);
    for (int l = c * per + (int)(xcd ? blockIdx.x >> 3 : blockIdx.x); l < l1; l += nl) {
      int tm, tn;
      tri_tile(l, p.upper_only != 0, &tm, &tn);
      if (p.tria == TRI_NONE && p.trib == TRI_NONE) bb_tile<CF, false>(p, tm, tn, smem_bb);
      else bb_tile<CF, true>(p, tm, tn, smem_bb);
      __syncthreads();
    }
  } else if ((gridDim.x & 7) == 0 && p.tria == TRI_NONE && p.trib == TRI_NONE) {
    const int c = blockIdx.x & 7, nl = gridDim.x >> 3;
    const int per = (tiles + 7) >> 3;
    const int l1 = min(tiles, (c + 1) * per);
    for (int l = c * per + (int)(blockIdx.x >> 3); l < l1; l += nl) {
      const int g = l / (XCD_GM * tiles_n);              // band of tile rows
      const int rows = min(XCD_GM, tiles_m - g * XCD_GM);
      const int r = l - g * XCD_GM * tiles_n;
      bb_tile<CF, false>(p, g * XCD_GM + r % rows, r / rows, smem_bb);
      __syncthreads();   // the LDS ring is reused by the next tile
    }
  } else {
    for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
      int tm, tn;
      tile_order(tile, tiles_m, tiles_n, p.tria, p.trib, &tm, &tn);
      if (p.tria == TRI_NONE && p.trib == TRI_NONE) bb_tile<CF, false>(p, tm, tn, smem_bb);
      else bb_tile<CF, true>(p, tm, tn, smem_bb);
      __syncthreads();
    }
  }
}

}  // namespace

int gemm_bb_tile(bool mid) { return mid ? MidCfg::BM : BigCfg::BM; }
int gemm_bb_bk() { return BK; }

void launch_gemm_bb(hipStream_t s, dim3 grid, const GemmParams& p, bool mid) {
  if (mid)
    hipLaunchKernelGGL(gemm_bb_kernel<MidCfg>, grid, dim3(MidCfg::NTH), 0, s, p);
  else
    hipLaunchKernelGGL(gemm_bb_kernel<BigCfg>, grid, dim3(BigCfg::NTH), 0, s, p);
}

}  // namespace ifk
