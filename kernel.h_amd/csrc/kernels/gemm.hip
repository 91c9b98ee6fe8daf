// fp32 GEMM for gfx950 on the matrix cores: C[m,n] = A[m,k] B[k,n],
// row-major, v_mfma_f32_32x32x2f32.
//
// Symbol and memref arguments follow the reference template
// (lib/dsl/kernels/gemm.cpp:116-296): A [m,k], B [k,n], C [m,n], rank 2,
// 21 parameters. The reference computes one element per lane with scalar
// FMAs out of an 8 KiB LDS tile (gemm.cpp:265-296). Here:
//
//   * Workgroup = 256 threads (4 wave64s, 2x2) computing a BM x BN tile of C;
//     each wave owns a quarter as WTM x WTN MFMA 32x32 accumulators. Four
//     symbols, all correct for every shape; the launcher scores each by its
//     full-occupancy rate times how busy its last round of workgroups would
//     be (kh_tiles.h) and takes the best:
//       `gemm`        128x256 tiles (64x128 per wave, 128 accumulator registers
//                     per lane), 16-deep K slabs: the least LDS and L2 traffic
//                     per MFMA (8192^3, 4096^3, 8192x8192x256); persistent
//                     workgroups, two per CU, each looping over its tiles;
//       `gemm_mid`    128x128 tiles (64x64 per wave), 32-deep slabs (e.g.
//                     8192x1024x8192);
//       `gemm_small`  64x64 tiles, for grids the larger tiles would fill
//                     unevenly (512^3, 1024^3);
//       `gemm_small_pf2` the same tiles with two-ahead prefetch, when they
//                     number at least KH_GEMM_SMALL_PF2_TILES (2048^3 to
//                     3584^3, 6144x6144x1024).
//     Registers are capped for two waves per SIMD (two workgroups per CU, as
//     LDS allows), so one workgroup's barrier and slab hand-over overlap the
//     other's MFMAs. `gemm` and `gemm_mid` raise their waves' priority
//     (s_setprio) while they issue MFMAs, so a wave that is feeding the
//     matrix core wins issue over one that is between slabs (+2% each).
//   * K advances in slabs staged through LDS. `gemm` loads its slabs straight
//     into LDS (buffer_load_dwordx4 ... lds) through three stages: slab ks+2
//     is in flight while slab ks is consumed, and the one barrier per slab sits
//     after the slab's first 8-deep chunk, so the next slab's first fragments
//     are read while the rest of this one feeds the MFMAs. Against staging the
//     slab through registers and ds_write (still used by `gemm_mid` and
//     `gemm_small`, where it measured as fast) that is +2% at 8192^3: the
//     stores and the wait for them sat between a wave's last MFMA of one slab
//     and its first of the next.
//   * LDS holds A as [m][k] (one ds_read_b128 per lane delivers four k
//     values) and B as [k][n] (a half-wave reads 32 consecutive n with
//     ds_read_b32), both conflict-free: rows padded by 4 floats when slabs are
//     staged through registers; for direct-to-LDS slabs, whose loads write 64
//     float4s contiguously, A's rows are unpadded with their float4s
//     XOR-swizzled and B's rows padded per group a wave loads. Slab loads are
//     branch-free buffer loads for aligned operands with k, n multiples of 4;
//     their range checks zero-fill the tails (the guarded per-element form of
//     the generic path made the compiler split every load into branches and
//     dword pieces, which cost 15% of the MFMA rate).
//   * K order inside an MFMA: the instruction sums k over its two lane
//     halves, and any permutation of k applied to both operands gives the
//     same product. Lane half h reads k = 8c + 4h + {0..3}; MFMA step s of
//     chunk c consumes k = 8c + s (half 0) and 8c + 4 + s (half 1).
//   * Tiles are ordered for the 8 XCDs (each with its own L2): consecutive
//     workgroups go round-robin to XCDs, so the launch index is remapped to
//     give every XCD a contiguous range of tiles, grouped 8 tile-rows deep
//     so neighbouring workgroups share A rows and B columns in L2.
//
// Tails in m, n and k are zero-filled on load and guarded on store, so any
// shape is correct; tiles are grid-strided so any grid is correct, including
// the reference's ceil(m/32) x 256 geometry (kernelh_backend.cpp:225).
// Accumulation is fp32 throughout (the MFMA accumulates in fp32).
#include "gemm_tiles.h"

using khg::Tile;
using khg::gemm_entry;
using khg::kThreads;

static_assert(Tile<2, 4, 16, true>::BM == KH_GEMM_BM && Tile<2, 4, 16, true>::BN == KH_GEMM_BN, "launcher tile size");
static_assert(Tile<2, 2, 32, false>::BM == KH_GEMM_MID_BM && Tile<2, 2, 32, false>::BN == KH_GEMM_MID_BN,
              "launcher tile size");
static_assert(Tile<1, 1, 32, false>::BM == KH_GEMM_SMALL_BM && Tile<1, 1, 32, false>::BN == KH_GEMM_SMALL_BN &&
                  Tile<1, 1, 16, false>::BM == KH_GEMM_SMALL_BM && Tile<1, 1, 16, false>::BN == KH_GEMM_SMALL_BN,
              "launcher tile size (gemm_small and gemm_small_pf2)");

// The reference symbol: 128x256 tiles, persistent. Each workgroup loops
// over tiles bid, bid + grid, ... (the launcher gives it min(tiles, two per
// CU) workgroups; any grid is correct) and the three-stage slab ring runs on
// across them, so a tile starts with its first two slabs already fetched.
// Against one tile per workgroup (the previous form of this symbol, same
// box): 8192^3 143.4 vs 142.0, 8192x8192x256 125.4 vs 123.0 TFLOP/s. Writing C
// as float4s (MFMA operands swapped so a lane holds four consecutive
// columns) let the stores overlap the next tile, but its 32-byte row pieces
// doubled the kernel's L2 misses and measured 0.7% slower at 8192^3; C goes
// out as whole 128-byte lines. K <= 16 and unaligned operands take the
// per-tile pipeline (or the generic path).
extern "C" __global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
gemm(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B), KH_MEMREF2(float, C)) {
  khg::gemm_entry_flat<2, 4, 16, true>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0, B_n1, A_n1, A_s0, B_s0, C_s0);
}

// Same arguments and results with 128x128 tiles.
extern "C" __global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
gemm_mid(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B), KH_MEMREF2(float, C)) {
  gemm_entry<2, 2, 32, true, false>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0, B_n1, A_n1, A_s0, B_s0, C_s0);
}

// Same arguments and results with 64x64 tiles.
extern "C" __global__ void __launch_bounds__(kThreads)
gemm_small(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B), KH_MEMREF2(float, C)) {
  gemm_entry<1, 1, 32, false, false>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0, B_n1, A_n1, A_s0, B_s0, C_s0);
}

// Same arguments and results with 64x64 tiles, 16-deep slabs prefetched two
// ahead through registers: more loads in flight per CU, for grids of many
// tiles (+5-7% over `gemm_small` from six tiles per CU, 2560^3 to
// 6144x6144x1024). With one or two tiles per CU the fewer barriers of
// `gemm_small`'s 32-deep slabs win (1024^3: 77 vs 71 TFLOP/s). A kernel of its
// own: compiled into `gemm_small` behind a size test, both pipelines lost 4%.
extern "C" __global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
gemm_small_pf2(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B), KH_MEMREF2(float, C)) {
  khg::gemm_entry_pipe<1, 1, 16, false, khg::kPipePrefetch2>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0, B_n1, A_n1, A_s0,
                                                             B_s0, C_s0);
}

