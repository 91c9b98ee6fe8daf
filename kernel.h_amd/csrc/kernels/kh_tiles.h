// Tile constants shared by the gfx950 kernels and the host launcher's
// geometry (khrt_templates.cpp). Plain macros: included by device and host
// translation units alike.
#pragma once

// Elementwise kernels (vecadd, fused_gelu): dwordx4 vectors per thread per
// grid-stride step.
#define KH_EW_UNROLL 4

// Scan: workgroup size chosen by the launcher (the kernel accepts 256..1024);
// each thread owns 16 elements, so a tile is 16 x KH_SCAN_THREADS elements.
#define KH_SCAN_THREADS 1024
#define KH_SCAN_TILE (16 * KH_SCAN_THREADS)

// GEMM block tile (rows of C x columns of C per workgroup of 256 threads).
#define KH_GEMM_BM 128
#define KH_GEMM_BN 128

// Attention: query rows per workgroup (4 wavefronts x 32 rows).
#define KH_ATTN_BLOCK_Q 128
