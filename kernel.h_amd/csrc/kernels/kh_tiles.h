// Tile constants shared by the gfx950 kernels and the host launcher's
// geometry (khrt_templates.cpp). Plain macros: included by device and host
// translation units alike.
#pragma once

// Elementwise kernels (vecadd, fused_gelu): dwordx4 vectors per thread per
// grid-stride step.
#define KH_EW_UNROLL 4

// Scan: workgroup size chosen by the launcher (the kernel accepts 256..1024).
// One wave of each workgroup runs the look-back; every other thread owns
// KH_SCAN_PER_THREAD consecutive elements, so a tile is
// KH_SCAN_PER_THREAD x (threads - 64) elements.
#ifndef KH_SCAN_PER_THREAD
#define KH_SCAN_PER_THREAD 16
#endif
#define KH_SCAN_THREADS 1024
#define KH_SCAN_TILE (KH_SCAN_PER_THREAD * (KH_SCAN_THREADS - 64))
// The launcher's workgroup size up to KH_SCAN_SMALL_N elements: at
// n = 10^6, 89 tiles of 11,264 ran 8.35 us against 66 of 15,360 in
// 8.52 us; at 2 * 10^6 1024 threads were faster (10.1 against 10.6 us).
#define KH_SCAN_SMALL_THREADS 768
#define KH_SCAN_SMALL_N (3 << 19)

// GEMM block tiles (rows of C x columns of C per workgroup of 256 threads).
#define KH_GEMM_BM 128
#define KH_GEMM_BN 256
#define KH_GEMM_MID_BM 128
#define KH_GEMM_MID_BN 128
#define KH_GEMM_SMALL_BM 64
#define KH_GEMM_SMALL_BN 64
// `gemm_small` runs eight waves (512 threads), two workgroups per CU.
#define KH_GEMM_SMALL_THREADS 512
// `gemm_wide`: 128x128 tiles on eight waves (512 threads), one workgroup per
// CU, persistent.
#define KH_GEMM_WIDE_BM 128
#define KH_GEMM_WIDE_BN 128
#define KH_GEMM_WIDE_THREADS 512

// The launcher's tile choice (khrt_templates.cpp, heuristic_gemm_symbol):
// for each symbol, score = its measured rate at full occupancy (TFLOP/s,
// MI355X) x the fraction of the last round of workgroups that is busy, and
// take the best. `gemm` and `gemm_mid` run two workgroups per CU, so a round
// is 2 x KH_GEMM_CUS tiles and a half-empty last round costs a full one;
// `gemm_wide` runs one per CU (a round of KH_GEMM_CUS tiles); the 64x64
// tiles (`gemm_small`, persistent, two per CU) are light enough that a
// partial round costs little, so their rounds are counted per CU. Fitted on 20 shapes from 1024^3 to 8192^3 (square,
// skinny, rectangular, deep K) timed with rotated U[-1,1] inputs and warm
// clocks: the choice is the measured best or within 3% of it on all of them.
// `gemm_wide`'s rate was refitted when it became the persistent 128x128
// ring: 3.3% below `gemm` at 4096^3 (both in whole rounds), level with the
// 64x64 tiles at 2560^3. Its round divides `gemm_mid`'s and its rate is
// higher, so it outscores `gemm_mid` at every shape (measured 5-6% faster
// at 4096x2048x4096 and 8192x1024x8192).
#define KH_GEMM_CUS 256
#define KH_GEMM_ROUND_BIG (2 * KH_GEMM_CUS)
#define KH_GEMM_ROUND_MID (2 * KH_GEMM_CUS)
#define KH_GEMM_ROUND_WIDE KH_GEMM_CUS
#define KH_GEMM_ROUND_SMALL KH_GEMM_CUS
#define KH_GEMM_RATE_BIG 142
#define KH_GEMM_RATE_MID 135
#define KH_GEMM_RATE_WIDE 137
#define KH_GEMM_RATE_SMALL 126
// `gemm_ksplit`: 32x32 tiles, K split over the 8 waves of a 512-thread
// workgroup. The launcher takes it when its tiles fit one round (at most
// one workgroup per CU): there the larger tiles leave three CUs in four idle.
// It also takes it where the 64x64 tiles number fewer than the CUs and
// every 32x32 tile is whole with K a multiple of KH_GEMM_KSPLIT_INTERIOR_K
// (the K-split symbols' unconditional-load path), from
// KH_GEMM_KSPLIT_MIN_K on; the workgroups then loop over their tiles.
// Kernel trace, rotated inputs, against the four-wave register-staged
// 64x64 tiles `gemm_small` then had: 640^3 11.5 vs 18.0 us, 768^3 18.0 vs
// 21.2, 1024x512x512 10.2 vs 15.2, 256x2048x2048 25.5 vs 50.3,
// 512x1536x1024 21.5 vs 27.4; level at 768x768x256 and 896^3; at 1024^3
// (256 tiles of 64x64) level, at 1024x1024x512 slower (17.3 vs 15.9).
// Against the persistent eight-wave `gemm_small`: 768^3 level (18.0 vs
// 17.8), 512x512x2048 14.6 vs 40.4.
#define KH_GEMM_KSPLIT_BM 32
#define KH_GEMM_KSPLIT_BN 32
#define KH_GEMM_KSPLIT_THREADS 512
#define KH_GEMM_KSPLIT_INTERIOR_K 128
#define KH_GEMM_KSPLIT_MIN_K 256
// From this K on, the launcher takes `gemm_ksplit_deep` (three batches of
// loads in flight per wave) for the same launches.
#define KH_GEMM_KSPLIT_DEEP_K 2048

// Attention: query rows per workgroup (4 wavefronts x 32 rows).
#define KH_ATTN_BLOCK_Q 128
