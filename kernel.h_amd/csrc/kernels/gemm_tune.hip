// GEMM tune candidates for `kernelh tune`: one kernel per entry of
// KH_GEMM_TUNE_CONFIGS, each with the template `gemm` arguments
// (A [m,k], B [k,n], C [m,n]; 21 parameters) and results, built from the
// same blocks as the product kernels (gemm_tiles.h). Embedded in the CLI,
// not in the product library.
#include "gemm_tiles.h"
#include "gemm_tune_list.h"

#define KH_GEMM_TUNE_KERNEL(WTM, WTN, BK, PRIO, DMA)                                                      \
  extern "C" __global__ void __launch_bounds__(khg::kThreads) __attribute__((amdgpu_waves_per_eu(2)))    \
  KH_GEMM_TUNE_SYMBOL(WTM, WTN, BK, PRIO, DMA)(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B),  \
                                               KH_MEMREF2(float, C)) {                                  \
    khg::gemm_entry<WTM, WTN, BK, PRIO != 0, DMA != 0>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0, B_n1, A_n1, \
                                                       A_s0, B_s0, C_s0);                                \
  }

KH_GEMM_TUNE_CONFIGS(KH_GEMM_TUNE_KERNEL)
