// fp32 GEMM for gfx950 on the matrix cores: C[m,n] = A[m,k] B[k,n],
// row-major, v_mfma_f32_32x32x2f32 (and v_mfma_f32_16x16x4f32 for the
// 64x64-tile pipelines where it measured faster).
//
// Symbol and memref arguments follow the reference template
// (lib/dsl/kernels/gemm.cpp:116-296): A [m,k], B [k,n], C [m,n], rank 2,
// 21 parameters. The reference computes one element per lane with scalar
// FMAs out of an 8 KiB LDS tile (gemm.cpp:265-296). Here:
//
//   * Workgroup = 256 threads (4 wave64s, 2x2; `gemm_wide`: 512, 4x2)
//     computing a BM x BN tile of C; each wave owns its part as WTM x WTN
//     MFMA accumulator blocks. Five such symbols, all correct for every
//     shape; the launcher scores each by its full-occupancy rate times how
//     busy its last round of workgroups would be (kh_tiles.h) and takes the
//     best, unless the launch has at most 256 tiles of 32x32, or fewer
//     than 256 tiles of 64x64 that are all whole with K a multiple of 128
//     (then `gemm_ksplit` / `gemm_ksplit_deep`, at the end of this file,
//     split K over 8 waves instead); a tune cache, when set, overrides the
//     choice:
//       `gemm`        128x256 tiles (64x128 per wave, 128 accumulator registers
//                     per lane), 16-deep K slabs: the least LDS and L2 traffic
//                     per MFMA (8192^3, 4096^3, 8192x8192x256); persistent
//                     workgroups, two per CU, each looping over its tiles;
//       `gemm_mid`    128x128 tiles (64x64 per wave), 32-deep slabs (the
//                     tune cache's; `gemm_wide` outscores it wherever both
//                     fit);
//       `gemm_small`  64x64 tiles on eight waves of 16x16 MFMAs (16x32 per
//                     wave) in the persistent direct-to-LDS ring, two
//                     workgroups per CU, for grids the larger tiles would
//                     fill unevenly (1024^3, 960^3, 1536^3 to 3584^3);
//       `gemm_small_pf2` 64x64 tiles on four waves of 16x16 MFMAs with
//                     two-ahead register prefetch (the tune cache's);
//       `gemm_wide`   128x128 tiles on eight waves of 16x16 MFMAs (32x64
//                     per wave), 32-deep slabs in `gemm`'s persistent
//                     direct-to-LDS ring, one workgroup per CU, where its
//                     tiles fill whole rounds (2048^3, 6144x6144x1024,
//                     2048x2048x8192, 4096x2048x4096, 8192x1024x8192).
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
//     `gemm_small_pf2`) that is +2% at 8192^3: the
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
static_assert(Tile<1, 2, 32, true, 4, 2, 16>::BM == KH_GEMM_SMALL_BM &&
                  Tile<1, 2, 32, true, 4, 2, 16>::BN == KH_GEMM_SMALL_BN &&
                  Tile<1, 2, 32, true, 4, 2, 16>::NT == KH_GEMM_SMALL_THREADS &&
                  Tile<2, 2, 32, false, 2, 2, 16>::BM == KH_GEMM_SMALL_BM &&
                  Tile<2, 2, 32, false, 2, 2, 16>::BN == KH_GEMM_SMALL_BN,
              "launcher tile size (gemm_small and gemm_small_pf2)");
static_assert(Tile<2, 4, 32, true, 4, 2, 16>::BM == KH_GEMM_WIDE_BM &&
                  Tile<2, 4, 32, true, 4, 2, 16>::BN == KH_GEMM_WIDE_BN &&
                  Tile<2, 4, 32, true, 4, 2, 16>::NT == KH_GEMM_WIDE_THREADS,
              "launcher tile size (gemm_wide)");

// Entry of a symbol whose tile split assumes THREADS one-dimensional
// threads per workgroup: the arguments in one round, then any other launch
// shape refused by writing NaN over C (khg::refuse_launch) instead of
// computing part of each tile.
#define KH_GEMM_ENTRY_CHECK(THREADS)                                                                            \
  const uint32_t gxy = kh::group_size_word(), gz = kh::group_size_z_word();                                   \
  KH_GEMM_ARGS_READY(gxy, gz);                                                                                 \
  if (kh::threads_x_of(gxy) != (THREADS) || kh::threads_y_of(gxy) != 1 || kh::threads_z_of(gz) != 1) {       \
    khg::refuse_launch(KH_PTR(C), C_n0, C_n1, C_s0);                                                           \
    return;                                                                                                    \
  }

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
  KH_GEMM_ENTRY_CHECK(kThreads);
  khg::gemm_entry_flat<2, 4, 16, true>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0, B_n1, A_n1, A_s0, B_s0, C_s0);
}

// Same arguments and results with 128x128 tiles.
extern "C" __global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
gemm_mid(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B), KH_MEMREF2(float, C)) {
  KH_GEMM_ENTRY_CHECK(kThreads);
  gemm_entry<2, 2, 32, true, false>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0, B_n1, A_n1, A_s0, B_s0, C_s0);
}

// Same arguments and results with 64x64 tiles on eight waves (4 x 2, each
// 16x32 as 1x2 blocks of v_mfma_f32_16x16x4f32), 32-deep slabs through
// `gemm`'s persistent direct-to-LDS ring; 49.5 KB of LDS and 86 VGPRs, so
// two workgroups per CU. Kernel trace, interleaved launches, same bits,
// against the 64x64 tiles it replaced (four waves, register-staged
// slabs; and `gemm_small_pf2` where that was the launcher's choice):
// 1024^3 28.2 -> 23.7 us, 1024x1024x512 16.3 -> 13.5-14.9,
// 1024x1024x8192 201.5 -> 160.9, 1536^3 86.8 -> 83.6, 2048x1024x1024 45.0
// -> 41.9, 2560^3-3584^3 within 1.3%. One workgroup per CU: 1536^3 91.0.
// The tile split assumes 512 threads: any other launch is refused by
// writing NaN over C.
extern "C" __global__ void __launch_bounds__(KH_GEMM_SMALL_THREADS) __attribute__((amdgpu_waves_per_eu(2)))
gemm_small(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B), KH_MEMREF2(float, C)) {
  KH_GEMM_ENTRY_CHECK(KH_GEMM_SMALL_THREADS);
  khg::gemm_entry_flat<1, 2, 32, true, 4, 2, 16>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0, B_n1, A_n1, A_s0, B_s0,
                                                 C_s0);
}

// Same arguments and results with 64x64 tiles on v_mfma_f32_16x16x4f32 (each
// wave 32x32 as 2x2 blocks of 16x16), 32-deep slabs prefetched two ahead
// through registers: more loads in flight per CU, for grids of many tiles.
// The tune space found the 16x16 form faster than the same tiles on 32x32
// MFMAs at every shape timed (rotated U[-1,1] inputs, warm clocks): 2048^3
// 121.5 vs 117.0, 3072^3 123.4 vs 114.2, 2048x2048x8192 127.6 vs 108.1,
// 6144x6144x1024 125.0 vs 121.1 TFLOP/s; level at 1536^3. The persistent
// eight-wave `gemm_small` has since matched or beaten it at every shape
// timed, so the launcher no longer picks it; a tune cache can.
extern "C" __global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
gemm_small_pf2(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B), KH_MEMREF2(float, C)) {
  KH_GEMM_ENTRY_CHECK(kThreads);
  khg::gemm_entry_pipe<2, 2, 32, true, khg::kPipePrefetch2, 2, 2, 16>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0, B_n1,
                                                                      A_n1, A_s0, B_s0, C_s0);
}

// Same arguments and results with 128x128 tiles on eight waves (4 x 2,
// each 32x64 as 2x4 blocks of v_mfma_f32_16x16x4f32), 32-deep slabs through
// `gemm`'s persistent three-stage direct-to-LDS ring (99 KB of LDS: one
// workgroup per CU, two waves per SIMD). Kernel trace against the previous
// `gemm_wide` (64x128 tiles, register-staged slabs), variants interleaved
// launch by launch, same bits: 2048^3 145.2 -> 133.9 us, 6144x6144x1024
// 586.5 -> 557.1, 2048x2048x8192 528.8 -> 487.1; and against `gemm_mid` at
// 4096x2048x4096 529.3 -> 496.9, 8192x1024x8192 1018 -> 965. The same tile
// with the waves 2 x 4 (64x32 each) ran 137.6 us at 2048^3, sixteen waves
// 140.5, 64x128 tiles two per CU 137.8, without s_setprio 137.0. The tile
// split assumes 512 threads: any other launch is refused by writing NaN
// over C.
extern "C" __global__ void __launch_bounds__(KH_GEMM_WIDE_THREADS) __attribute__((amdgpu_waves_per_eu(2)))
gemm_wide(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B), KH_MEMREF2(float, C)) {
  KH_GEMM_ENTRY_CHECK(KH_GEMM_WIDE_THREADS);
  khg::gemm_entry_flat<2, 4, 32, true, 4, 2, 16>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0, B_n1, A_n1, A_s0, B_s0,
                                                 C_s0);
}


// 32x32 tiles with K split over the workgroup's waves (8 at the launcher's
// 512 threads; any 64..512 threads, a multiple of 64, are correct), for
// launches whose larger tiles leave most CUs idle: 512^3 has 64 tiles of
// 64x64 for 256 CUs, and 256 tiles of 32x32. Wave w of nw accumulates the
// products of its K range (contiguous chunks of kc = 8 * ceil(K / (8 nw)))
// straight from global memory into one v_mfma_f32_32x32x2f32 accumulator,
// without LDS: lane l (r = l % 32, h = l / 32) loads the float4
// A[m0 + r][k + 4h .. k + 4h + 3] and the four B[k + 4h + i][n0 + r], so MFMA
// i of a group of 8 k sums k + i (lanes 0-31) and k + 4 + i (lanes 32-63):
// every k of the group exactly once. Rows, columns and k past the matrix or
// chunk edge load a clamped in-range address and are replaced by 0, so the
// loads carry no branch. The partial tiles meet in LDS, and output register
// i is summed by wave i % nw in the fixed order w0 + w1 + ... : the result
// does not depend on timing. Measured against `gemm_small` (64x64 tiles):
// 512^3 28-30 vs 18.0 TFLOP/s, 512x512x2048 37-41 vs 22, 256^3 6.3-6.5 vs
// 3.8. Four waves per workgroup reached 22 at 512^3; sixteen spilled, and
// so did loading 8 groups per batch (6 groups: slower at every shape).
//
// Where every tile is whole and every wave's K chunk a whole number of
// batches (M, N multiples of 32, K of 128, 512 threads: the BASELINE 512^3),
// the kernel takes a path of its own before the general one (ks_interior):
// buffer loads with one offset register per operand and lane and the k step
// in the scalar offset, none of them conditional. In the general path the
// compiler turns each "clamped load, then select 0" into a branch around the
// load and waits for it where the branches join, so a wave's loads went out
// one at a time. Kernel trace, rotated inputs, same bits: 512^3 9.8 -> 6.2
// us, 512x512x1024 16.4 -> 9.0, 256^3 5.7 -> 4.5; and, in the deep symbol,
// 512x512x2048 25.6 -> 14.4, 512x512x8192 82 -> 49. Batches of 2 groups,
// two sets in flight, measured best (4 groups: 6.8 us at 512^3, 8: 7.7;
// three sets: 6.7).
namespace {

using khg::v16f;
using kh::u32x4_t;
constexpr int kKsTile = KH_GEMM_KSPLIT_BM;
constexpr int kKsMaxWaves = KH_GEMM_KSPLIT_THREADS / 64;
constexpr int kKsBatch = 4;  // groups of 8 k loaded ahead per batch
constexpr int kKsFastBatch = 2;  // the same, in ks_interior
static_assert(KH_GEMM_KSPLIT_BM == 32 && KH_GEMM_KSPLIT_BN == 32, "one 32x32 MFMA accumulator per wave");

// Loads one group of 8 k for this lane: k is the lane's first k of the
// group (a multiple of 4 when VEC), K the end of the wave's chunk.
template <bool VEC>
__device__ __forceinline__ void ks_load(const float *__restrict__ A, const float *__restrict__ B, int64_t K,
                                        int64_t lda, int64_t ldb, int64_t arow, int64_t bcol, bool arow_ok,
                                        bool bcol_ok, int64_t k, float4 &a, float (&b)[4]) {
  if constexpr (VEC) {
    const bool ok = arow_ok && k < K;
    const float4 t = *reinterpret_cast<const float4 *>(A + arow * lda + (k < K ? k : K - 4));
    a = ok ? t : make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t kk = k + i;
      const float v = A[arow * lda + (kk < K ? kk : K - 1)];
      t[i] = (arow_ok && kk < K) ? v : 0.0f;
    }
    a = make_float4(t[0], t[1], t[2], t[3]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t kk = k + i;
    const float v = B[(kk < K ? kk : K - 1) * ldb + bcol];
    b[i] = (bcol_ok && kk < K) ? v : 0.0f;
  }
}

__device__ __forceinline__ void ks_mfma(v16f &acc, const float4 &a, const float (&b)[4]) {
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b[3], acc, 0, 0, 0);
}

// NWC: the wave count when known at compile time (the launcher's 512
// threads), else 0 and the count comes from blockDim. DEEP compiles in the
// interior-tile path with three batches of loads in flight, for K chunks of
// at least three batches.
template <bool VEC, int NWC, bool DEEP>
__device__ __forceinline__ void gemm_ksplit_body(const float *__restrict__ A, const float *__restrict__ B,
                                                 float *__restrict__ C, int64_t M, int64_t N, int64_t K,
                                                 int64_t lda, int64_t ldb, int64_t ldc, int bd, int64_t nblocks,
                                                 float *red) {
  const int lane = kh::lane_id(), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kh::kWave);
  const int nw = NWC > 0 ? NWC : bd / kh::kWave;  // whole waves; a partial last wave takes no k, no output
  const int r = lane & 31, h = lane >> 5;
  const int64_t tiles_m = (M + kKsTile - 1) / kKsTile, tiles_n = (N + kKsTile - 1) / kKsTile;
  const int64_t total = tiles_m * tiles_n;
  // DEEP chunks are whole batches of 4 groups (32 k).
  const int64_t kc = DEEP ? 32 * ((K + 32 * nw - 1) / (32 * nw)) : 8 * ((K + 8 * nw - 1) / (8 * nw));
  const int64_t kb = wave * kc, ke = kb + kc < K ? kb + kc : K;
  const int64_t groups = ke > kb ? (ke - kb + 7) / 8 : 0;
  for (int64_t t = blockIdx.x; t < total; t += nblocks) {
    const int64_t m0 = (t / tiles_n) * kKsTile, n0 = (t % tiles_n) * kKsTile;
    const bool arow_ok = m0 + r < M, bcol_ok = n0 + r < N;
    const int64_t arow = arow_ok ? m0 + r : M - 1, bcol = bcol_ok ? n0 + r : N - 1;
    v16f acc = {};
    if (DEEP && VEC && m0 + kKsTile <= M && n0 + kKsTile <= N && ke - kb == kc && kc >= 3 * 32 &&
        31 * lda + 8 <= (1 << 30) && (kc + 8) * ldb + 32 <= (1 << 30)) {
      // Interior tile, a whole chunk of at least three batches: no clamps,
      // and three batches of loads in flight (a ring of three register
      // sets; the tail reloads the last batch and skips its math).
      const uint32_t aoff = (uint32_t)(r * lda + 4 * h), boff = (uint32_t)(4 * h * ldb + r);
      const float *abase = A + m0 * lda + kb, *bbase = B + kb * ldb + n0;
      const int64_t nb = kc / 32;
      struct Set {
        float4 a[kKsBatch];
        float b[kKsBatch][4];
      };
      Set f0, f1, f2;
      auto fload = [&](Set &f, int64_t j) {
#pragma unroll
        for (int i = 0; i < kKsBatch; ++i) {
          f.a[i] = *reinterpret_cast<const float4 *>(abase + (32 * j + 8 * i) + aoff);
#pragma unroll
          for (int q = 0; q < 4; ++q) f.b[i][q] = (bbase + (32 * j + 8 * i + q) * ldb)[boff];
        }
      };
      auto fmath = [&](const Set &f) {
#pragma unroll
        for (int i = 0; i < kKsBatch; ++i) ks_mfma(acc, f.a[i], f.b[i]);
      };
      fload(f0, 0);
      fload(f1, 1);
      for (int64_t j = 0; j < nb; j += 3) {
        fload(f2, j + 2 < nb ? j + 2 : nb - 1);
        fmath(f0);
        fload(f0, j + 3 < nb ? j + 3 : nb - 1);
        if (j + 1 < nb) fmath(f1);
        fload(f1, j + 4 < nb ? j + 4 : nb - 1);
        if (j + 2 < nb) fmath(f2);
      }
    } else {
    float4 a0[kKsBatch], a1[kKsBatch];
    float b0[kKsBatch][4], b1[kKsBatch][4];
    auto load = [&](float4 (&a)[kKsBatch], float (&b)[kKsBatch][4], int64_t g) {
#pragma unroll
      for (int i = 0; i < kKsBatch; ++i) {
        ks_load<VEC>(A, B, ke, lda, ldb, arow, bcol, arow_ok, bcol_ok, kb + 8 * (g + i) + 4 * h, a[i], b[i]);
      }
    };
    auto math = [&](const float4 (&a)[kKsBatch], const float (&b)[kKsBatch][4]) {
#pragma unroll
      for (int i = 0; i < kKsBatch; ++i) ks_mfma(acc, a[i], b[i]);
    };
    // Batches of kKsBatch groups, double-buffered: the next batch's loads
    // are issued before this batch's MFMAs. Groups past `groups` load
    // clamped addresses and contribute 0.
    if (groups > 0) load(a0, b0, 0);
    int64_t g = 0;
    for (; g + kKsBatch < groups; g += 2 * kKsBatch) {
      load(a1, b1, g + kKsBatch);
      math(a0, b0);
      if (g + 2 * kKsBatch < groups) load(a0, b0, g + 2 * kKsBatch);
      math(a1, b1);
    }
    if (g < groups) math(a0, b0);
    }
    // Partial tiles into LDS: red[wave][register][lane].
#pragma unroll
    for (int i = 0; i < 16; ++i) red[(wave * 16 + i) * kh::kWave + lane] = acc[i];
    kh::lds_barrier();
    if (wave < nw) {
      for (int i = wave; i < 16; i += nw) {
        float s = red[i * kh::kWave + lane];
        for (int w = 1; w < nw; ++w) s += red[(16 * w + i) * kh::kWave + lane];
        const int64_t gr = m0 + 8 * (i >> 2) + 4 * h + (i & 3), gc = n0 + r;
        if (gr < M && gc < N) C[gr * ldc + gc] = s;
      }
    }
    kh::lds_barrier();
  }
}

// A uniform pointer, forced into scalar registers: its computation may run
// on the vector ALU (the 64-bit multiply of a row index), and a buffer
// resource built from vector registers costs a loop around every load.
template <typename T>
__device__ __forceinline__ T *uniform_ptr(T *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T *>(((uint64_t)hi << 32) | lo);
}

// The K split for launches whose tiles are all whole: M, N multiples of 32,
// K of 8 * kKsFastBatch * 8, eight waves, and every buffer span below 2^31
// bytes, the largest record count a buffer resource holds (ks_interior_ok). The operands and groups are those of gemm_ksplit_body;
// lane (r, h) reads A from one offset register plus 32 bytes per group (the
// instruction's immediate) and B from one offset register plus a row step
// in the scalar offset. Same reduction, so the same bits.
__device__ __forceinline__ bool ks_interior_ok(int bd, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                               int64_t ldc, const float *A) {
  constexpr int64_t kLim = int64_t(1) << 29;
  static_assert(KH_GEMM_KSPLIT_INTERIOR_K == 64 * kKsFastBatch, "the launcher's K multiple for this path");
  return bd == KH_GEMM_KSPLIT_THREADS && M > 0 && N > 0 && (M & 31) == 0 && (N & 31) == 0 && K > 0 &&
         K % KH_GEMM_KSPLIT_INTERIOR_K == 0 && (lda & 3) == 0 && kh::aligned16(A) && M <= kLim && N <= kLim &&
         31 * lda + K / 8 < kLim && K * ldb < kLim && ldc < kLim && (M >> 5) * (N >> 5) < (int64_t(1) << 31);
}

__device__ __forceinline__ void ks_interior(const float *__restrict__ A, const float *__restrict__ B,
                                            float *__restrict__ C, int M, int N, int K, int lda, int ldb, int ldc,
                                            int nblocks, float *red) {
  constexpr int nw = kKsMaxWaves, NB = kKsFastBatch;
  const int lane = kh::lane_id(), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kh::kWave);
  const int r = lane & 31, h = lane >> 5;
  const int tiles_n = N / kKsTile, total = (M / kKsTile) * tiles_n;
  const int kc = K / nw, kb = wave * kc, nbat = kc / (8 * NB);
  const uint32_t va = (uint32_t)(4 * (r * lda + 4 * h)), vb = (uint32_t)(4 * (4 * h * ldb + r));
  const uint32_t bstep = (uint32_t)(4 * ldb);
  const uint32_t abytes = (uint32_t)(4 * (31 * lda + kc)), bbytes = (uint32_t)(4 * ((kc - 1) * ldb + kKsTile));
  struct Set {
    float4 a[NB];
    float b[NB][4];
  };
  for (int t = blockIdx.x; t < total; t += nblocks) {
    const int m0 = __builtin_amdgcn_readfirstlane((t / tiles_n) * kKsTile);
    const int n0 = __builtin_amdgcn_readfirstlane((t % tiles_n) * kKsTile);
    const __amdgpu_buffer_rsrc_t ra = kh::span_rsrc(uniform_ptr(A + (int64_t)m0 * lda + kb), abytes);
    const __amdgpu_buffer_rsrc_t rb = kh::span_rsrc(uniform_ptr(B + (int64_t)kb * ldb + n0), bbytes);
    v16f acc = {};
    Set s0, s1;
    auto load = [&](Set &s, int j) {
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int g = j * NB + i;
        const u32x4_t u = __builtin_amdgcn_raw_buffer_load_b128(ra, va, (uint32_t)(32 * g), 0);
        s.a[i] = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
#pragma unroll
        for (int q = 0; q < 4; ++q)
          s.b[i][q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, vb, (uint32_t)(8 * g + q) * bstep, 0));
      }
    };
    auto math = [&](const Set &s) {
#pragma unroll
      for (int i = 0; i < NB; ++i) ks_mfma(acc, s.a[i], s.b[i]);
    };
    // Two sets in flight: batch j + 1's loads go out before batch j's MFMAs.
    load(s0, 0);
    for (int j = 0; j < nbat; j += 2) {
      if (j + 1 < nbat) load(s1, j + 1);
      math(s0);
      if (j + 2 < nbat) load(s0, j + 2);
      if (j + 1 < nbat) math(s1);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) red[(wave * 16 + i) * kh::kWave + lane] = acc[i];
    kh::lds_barrier();
#pragma unroll
    for (int i = wave; i < 16; i += nw) {
      float s = red[i * kh::kWave + lane];
#pragma unroll
      for (int w = 1; w < nw; ++w) s += red[(16 * w + i) * kh::kWave + lane];
      C[(int64_t)(m0 + 8 * (i >> 2) + 4 * h + (i & 3)) * ldc + n0 + r] = s;
    }
    kh::lds_barrier();
  }
}

}  // namespace

template <bool DEEP>
__device__ __forceinline__ void gemm_ksplit_entry(const float *Ap, const float *Bp, float *Cp, int64_t M, int64_t N,
                                                  int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int bd,
                                                  int64_t nb, float *red) {
  const bool vec = ((K & 3) == 0) && ((lda & 3) == 0) && kh::aligned16(Ap);
  if (bd == KH_GEMM_KSPLIT_THREADS) {
    if (vec) {
      gemm_ksplit_body<true, kKsMaxWaves, DEEP>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, bd, nb, red);
    } else {
      gemm_ksplit_body<false, kKsMaxWaves, DEEP>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, bd, nb, red);
    }
  } else if (vec) {
    gemm_ksplit_body<true, 0, DEEP>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, bd, nb, red);
  } else {
    gemm_ksplit_body<false, 0, DEEP>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, bd, nb, red);
  }
}

// The arguments the K-split kernels use, loaded in one round (KH_ARGS_READY):
// at 512^3 the launch is ~10 us, and every serial round trip to
// kernel-argument memory before the first operand load is part of it.
#define KH_KSPLIT_ENTRY(DEEP)                                                                                  \
  const uint32_t gw = kh::group_size_word(), gz = kh::group_size_z_word(), nb = kh::grid_blocks_x();          \
  KH_ARGS_READY(A_base, A_off, A_n0, A_n1, A_s0, B_base, B_off, B_n1, B_s0, C_base, C_off, C_s0, gw, gz, nb); \
  if (kh::threads_y_of(gw) == 1 && kh::threads_z_of(gz) == 1 &&                                               \
      ks_interior_ok((int)kh::threads_x_of(gw), A_n0, B_n1, A_n1, A_s0, B_s0, C_s0, KH_PTR(A))) {             \
    ks_interior(KH_PTR(A), KH_PTR(B), KH_PTR(C), (int)A_n0, (int)B_n1, (int)A_n1, (int)A_s0, (int)B_s0,       \
                (int)C_s0, (int)nb, red);                                                                    \
    return;                                                                                                   \
  }                                                                                                           \
  gemm_ksplit_entry<DEEP>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0, B_n1, A_n1, A_s0, B_s0, C_s0,                \
                          (int)kh::threads_x_of(gw), nb, red)

extern "C" __global__ void __launch_bounds__(KH_GEMM_KSPLIT_THREADS)
gemm_ksplit(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B), KH_MEMREF2(float, C)) {
  __shared__ float red[kKsMaxWaves * 16 * 64];
  KH_KSPLIT_ENTRY(false);
}

// Same tiles and split with the deep-chunk path compiled in: the launcher
// takes it over `gemm_ksplit` for K >= KH_GEMM_KSPLIT_DEEP_K. A kernel of
// its own: compiled into `gemm_ksplit`, the extra registers slowed the
// short-chunk path (512^3: 28 -> 18 TFLOP/s). Measured against it:
// 512x512x2048 42 vs 37 TFLOP/s, 512x512x8192 54 vs 40; at K = 1024 the two
// were level.
extern "C" __global__ void __launch_bounds__(KH_GEMM_KSPLIT_THREADS)
gemm_ksplit_deep(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B), KH_MEMREF2(float, C)) {
  __shared__ float red[kKsMaxWaves * 16 * 64];
  KH_KSPLIT_ENTRY(true);
}
