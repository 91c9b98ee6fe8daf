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
// Smallest tile any accepted launch uses (256 threads); sizes the state.
#define KH_SCAN_MIN_TILE (KH_SCAN_PER_THREAD * (256 - 64))

// GEMM block tiles (rows of C x columns of C per workgroup of 256 threads).
// The launcher takes `gemm` (128x256) when its grid has at least
// KH_GEMM_TILES_256 tiles (two per CU on MI355X), else `gemm_mid` (128x128)
// when that grid has at least KH_GEMM_TILES_128 tiles, else `gemm_small`
// (64x64): the largest tile that still gives every CU work.
#define KH_GEMM_BM 128
#define KH_GEMM_BN 256
#define KH_GEMM_MID_BM 128
#define KH_GEMM_MID_BN 128
#define KH_GEMM_SMALL_BM 64
#define KH_GEMM_SMALL_BN 64
#define KH_GEMM_TILES_256 512
#define KH_GEMM_TILES_128 256

// Attention: query rows per workgroup (4 wavefronts x 32 rows).
#define KH_ATTN_BLOCK_Q 128
