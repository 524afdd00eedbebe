// Internal interface between the two GEMM kernels (gemm.hip, gemm_big.hip).
#pragma once
#include "gemm.h"

namespace ifk {

struct GemmParams {
  int64_t M, N, K;
  float alpha, beta;
  const void* A; int64_t lda; int tria; int64_t bsa;
  const void* B; int64_t ldb; int trib; int64_t bsb;
  float* C; int64_t ldc; int64_t bsc;
  bf16_t* Cb; int64_t ldcb; int64_t bscb;
  float* part;
  int splits;
  int tiles_m, tiles_n;
  int vec_a, vec_b;
  int vec_c;   // C (if any) 16-byte and Cb (if any) 8-byte aligned, with ld and
               // batch strides multiples of 4 elements: vector epilogue
  int upper_only;   // skip tiles wholly below the diagonal (square Gram output)
  int lower_only;   // skip tiles wholly above the diagonal
  // Stream-K (direct-to-LDS kernel, neither operand triangular; splits == 1):
  // sk_lanes > 0 lanes of tiles_n workgroups each (one per tile column) walk
  // an equal contiguous share of the (tile row, K slab) space of a batch
  // entry (grid.z), so every workgroup gets the same number of slabs however
  // few tiles there are.  A tile shared by several lanes is summed by the
  // last of them to arrive, in lane order, from the others' partial tiles.
  int sk_lanes;
  int sk_iters;     // K slabs per tile
  int* sk_cnt;      // arrival counter per tile and entry, zero at launch
  float* sk_part;   // partial tiles: two per lane, tile column and entry
};

// Lane of a stream-K walk over U (tile row, slab) steps with L lanes that
// holds step u: lane l covers [l U / L, (l + 1) U / L).
__host__ __device__ inline int sk_lane_of(int64_t u, int64_t U, int L) {
  return (int)(((u + 1) * (int64_t)L - 1) / U);
}

// Tile t of a grid-stride walk -> (tile row, tile column), heaviest tiles
// first when an operand is triangular: a tile's K range shrinks down the rows
// for an upper op(A) (up the rows for a lower one) and towards the left
// columns for an upper op(B) (the right ones for a lower one), and
// workgroups pick up tiles in order, so the longest ones start first.
// Without a triangular operand: column-major.
__device__ __forceinline__ void tile_order(int t, int tiles_m, int tiles_n, int tria, int trib,
                                           int* tm, int* tn) {
  if (tria == TRI_UPPER || tria == TRI_LOWER) {
    const int r = t / tiles_n;
    *tm = tria == TRI_UPPER ? r : tiles_m - 1 - r;
    *tn = t % tiles_n;
  } else if (trib == TRI_UPPER) {
    *tn = tiles_n - 1 - t / tiles_m;
    *tm = t % tiles_m;
  } else {
    *tm = t % tiles_m;
    *tn = t / tiles_m;
  }
}

// 256 x 256 x 32 bf16 kernel (gemm_big.hip); grid.x = tiles_m * tiles_n of
// its tile, grid.z = batch * splits.
int gemm_big_tile_m();
int gemm_big_tile_n();
int gemm_big_bk();
void launch_gemm_big(hipStream_t s, dim3 grid, const GemmParams& p, int adt, bool akc, int bdt,
                     bool bkc);

// bf16 x bf16 kernel for K-contiguous operands with a four-slab
// direct-to-LDS ring (gemm_bb.hip), square tile 256 (mid = false) or 128
// (mid = true), BK 32; grid.x = tiles, grid.z = batch * splits; in
// stream-K mode grid.x = sk_lanes * tiles_n (sk_lanes a multiple of 8) and
// grid.z = batch.
int gemm_bb_tile(bool mid);
int gemm_bb_bk();
void launch_gemm_bb(hipStream_t s, dim3 grid, const GemmParams& p, bool mid);

}  // namespace ifk
