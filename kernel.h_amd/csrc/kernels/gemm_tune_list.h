// The GEMM tune space for gfx950 (`kernelh tune`): wave tile WTM x WTN of
// 32x32 MFMA accumulators (workgroup = 2x2 waves, so 64 WTM x 64 WTN of C),
// K-slab depth BK, whether waves raise their priority while issuing MFMAs,
// and the slab pipeline (DMA 0: register-staged, two LDS stages; 1: loaded
// straight into three LDS stages). Pruned for wave64 and 160 KiB LDS: at most
// 8 accumulators per wave (two waves per SIMD fit in registers), every slab
// splits into whole float4s over 256 threads (BK = 8 needs both tile sides
// >= 128), and the three-stage pipeline only where its stages still let two
// workgroups share a CU. Shared by gemm_tune.hip (one kernel per entry) and
// the CLI (the candidate table), so the two cannot drift. 66 entries.
#pragma once

#define KH_GEMM_TUNE_CONFIGS(X) \
  X(1, 1, 16, 0, 0) X(1, 1, 16, 1, 0) X(1, 1, 16, 0, 1) X(1, 1, 16, 1, 1) \
  X(1, 1, 32, 0, 0) X(1, 1, 32, 1, 0) X(1, 1, 32, 0, 1) X(1, 1, 32, 1, 1) \
  X(1, 2, 16, 0, 0) X(1, 2, 16, 1, 0) X(1, 2, 16, 0, 1) X(1, 2, 16, 1, 1) \
  X(1, 2, 32, 0, 0) X(1, 2, 32, 1, 0) X(1, 2, 32, 0, 1) X(1, 2, 32, 1, 1) \
  X(2, 1, 16, 0, 0) X(2, 1, 16, 1, 0) X(2, 1, 16, 0, 1) X(2, 1, 16, 1, 1) \
  X(2, 1, 32, 0, 0) X(2, 1, 32, 1, 0) X(2, 1, 32, 0, 1) X(2, 1, 32, 1, 1) \
  X(2, 2, 8, 0, 0) X(2, 2, 8, 1, 0) X(2, 2, 8, 0, 1) X(2, 2, 8, 1, 1) \
  X(2, 2, 16, 0, 0) X(2, 2, 16, 1, 0) X(2, 2, 16, 0, 1) X(2, 2, 16, 1, 1) \
  X(2, 2, 32, 0, 0) X(2, 2, 32, 1, 0) \
  X(1, 4, 16, 0, 0) X(1, 4, 16, 1, 0) X(1, 4, 16, 0, 1) X(1, 4, 16, 1, 1) \
  X(1, 4, 32, 0, 0) X(1, 4, 32, 1, 0) \
  X(4, 1, 16, 0, 0) X(4, 1, 16, 1, 0) X(4, 1, 16, 0, 1) X(4, 1, 16, 1, 1) \
  X(4, 1, 32, 0, 0) X(4, 1, 32, 1, 0) \
  X(2, 4, 8, 0, 0) X(2, 4, 8, 1, 0) X(2, 4, 8, 0, 1) X(2, 4, 8, 1, 1) \
  X(2, 4, 16, 0, 0) X(2, 4, 16, 1, 0) X(2, 4, 16, 0, 1) X(2, 4, 16, 1, 1) \
  X(2, 4, 32, 0, 0) X(2, 4, 32, 1, 0) \
  X(4, 2, 8, 0, 0) X(4, 2, 8, 1, 0) X(4, 2, 8, 0, 1) X(4, 2, 8, 1, 1) \
  X(4, 2, 16, 0, 0) X(4, 2, 16, 1, 0) X(4, 2, 16, 0, 1) X(4, 2, 16, 1, 1) \
  X(4, 2, 32, 0, 0) X(4, 2, 32, 1, 0)

// Symbol of one candidate: gemm_t<WTM>x<WTN>_k<BK>_p<PRIO>_d<DMA>.
#define KH_GEMM_TUNE_SYMBOL(WTM, WTN, BK, PRIO, DMA) gemm_t##WTM##x##WTN##_k##BK##_p##PRIO##_d##DMA
