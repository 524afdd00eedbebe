// MFMA GEMM engine for gfx950: C = alpha * op(A) * op(B) + beta * C.
//
// op(A) is M x K and op(B) is K x N.  Each operand is described by where its
// K index runs in memory:
//   A.kc = true : op(A)[m][k] = A[m * ld + k]   (A stored M x K row-major)
//   A.kc = false: op(A)[m][k] = A[k * ld + m]   (A stored K x M, used transposed)
//   B.kc = true : op(B)[k][n] = B[n * ld + k]   (B stored N x K, used transposed)
//   B.kc = false: op(B)[k][n] = B[k * ld + n]   (B stored K x N row-major)
// Operands may be fp32 or bf16 in memory.  MATH_BF16 rounds them to bf16 (RNE)
// and runs v_mfma_f32_32x32x16_bf16; MATH_F32 keeps fp32 and runs
// v_mfma_f32_32x32x2f32.  Accumulation is fp32 in both.  A triangular flag on
// an operand both skips the K tiles that are structurally zero and masks the
// zero triangle on load, so the stored contents of that triangle never matter.
#pragma once
#include "common.h"

namespace ifk {

struct MatRef {
  const void* p;
  int dt;          // DT_F32 / DT_BF16
  int64_t ld;
  bool kc;         // see header comment
  int tri;         // TRI_NONE / TRI_UPPER / TRI_LOWER, describing op(X)
  int64_t bstride; // elements between batch entries
};

inline MatRef A_n(const void* p, int dt, int64_t ld, int tri = TRI_NONE, int64_t bs = 0) {
  return MatRef{p, dt, ld, true, tri, bs};
}
inline MatRef A_t(const void* p, int dt, int64_t ld, int tri = TRI_NONE, int64_t bs = 0) {
  return MatRef{p, dt, ld, false, tri, bs};
}
inline MatRef B_n(const void* p, int dt, int64_t ld, int tri = TRI_NONE, int64_t bs = 0) {
  return MatRef{p, dt, ld, false, tri, bs};
}
inline MatRef B_t(const void* p, int dt, int64_t ld, int tri = TRI_NONE, int64_t bs = 0) {
  return MatRef{p, dt, ld, true, tri, bs};
}

struct OutRef {
  float* c;        // fp32 output (may be null if cb is set and beta == 0)
  int64_t ldc;
  int64_t bstride;
  bf16_t* cb;      // optional RNE bf16 copy of the result
  int64_t ldcb;
  int64_t bstride_b;
  int upper = 0;   // only the upper triangle is wanted (a square Gram matrix):
                   // tiles wholly below the diagonal are skipped and hold
                   // unspecified values
  int lower = 0;   // only the lower triangle is wanted: tiles wholly above
                   // the diagonal (row index < column index throughout) are
                   // skipped and hold unspecified values
  int per_entry = 0;   // choose tile and split-K as for a single batch entry, so
                       // every entry of a batch gets the bits a batch of one gets
};

inline OutRef out_f32(float* c, int64_t ldc, int64_t bs = 0) {
  return OutRef{c, ldc, bs, nullptr, 0, 0};
}
inline OutRef out_bf16(bf16_t* cb, int64_t ld, int64_t bs = 0) {
  return OutRef{nullptr, 0, 0, cb, ld, bs};
}
inline OutRef out_both(float* c, int64_t ldc, bf16_t* cb, int64_t ldcb, int64_t bstride = 0,
                       int64_t bstride_b = 0) {
  return OutRef{c, ldc, bstride, cb, ldcb, bstride_b};
}
inline OutRef upper_part(OutRef o) {
  o.upper = 1;
  return o;
}
inline OutRef lower_part(OutRef o) {
  o.lower = 1;
  return o;
}
inline OutRef per_entry(OutRef o) {
  o.per_entry = 1;
  return o;
}

// Scratch the engine may use for split-K partial sums (fp32 elements).  When
// it is too small the engine uses fewer splits; it never fails for lack of it.
struct SplitScratch {
  float* p;
  size_t floats;
};

// Launch profiler (see gemm.hip).  variant: gemm_variant_id() (bit 5 set for
// the large-tile bf16 kernels, bit 6 as well for the direct-to-LDS one, bit 7
// for its 128 x 128 tile, bit 9 for a stream-K launch), -2 all, -3 all of the
// register-staged 256 x 128 kernel, -4 all of the 128 x 128 kernel, -5 / -6
// all of the direct-to-LDS kernel with its 256 / 128 tile, -7 / -8 all
// cholb_first / cholb_step launches, -1 off.
int gemm_variant_id(int math, int adt, bool akc, int bdt, bool bkc);
// The same profiler for other kernels: variant KVID + kind (families 5, 6:
// cholb_first_kernel, cholb_step_kernel; armed by -7 / -8).  A launcher
// brackets one launch with prof_kernel_begin / prof_kernel_end (no-ops when
// the profiler is not armed for it).
constexpr int KVID = 1 << 12;
constexpr int KVID_CHOLB_FIRST = KVID + 0, KVID_CHOLB_STEP = KVID + 1;
void* prof_kernel_begin(hipStream_t s, int vid, double flops, double bytes, int64_t m, int64_t n,
                        int64_t k);
void prof_kernel_end(void* rec, hipStream_t s);
int profile_begin(int variant);
int profile_end(int64_t* n_launches);
int profile_get(int64_t i, int* variant, float* ms, double* flops, double* bytes, int64_t* m,
                int64_t* n, int64_t* k);

// max_wgs > 0 caps the number of workgroups of a large-tile launch (tiles are
// then visited grid-stride, or a stream-K grid is sized within it), leaving
// CUs free for work on other streams.  Every product runs on this library's
// own kernels.
int gemm(hipStream_t s, int math, int64_t M, int64_t N, int64_t K, float alpha,
         const MatRef& A, const MatRef& B, float beta, const OutRef& C, int batch,
         SplitScratch scratch, int max_wgs = 0);

// Scratch (fp32 elements) that lets the GEMM of an M x N output with K deep
// operands take its fastest grid, stream-K included, for `batch` entries
// within max_wgs workgroups (0: uncapped).
size_t gemm_scratch_floats(int64_t M, int64_t N, int64_t K, int batch, int max_wgs = 0);

}  // namespace ifk
