// GEMM tune candidates for `kernelh tune` and for the launcher's tune cache:
// one kernel per entry of gemm_tune_list.h (the space and its prune rules
// are stated in gemm_tune_space.py), each with the template `gemm` arguments
// (A [m,k], B [k,n], C [m,n]; 21 parameters) and results, built from the
// same blocks as the product kernels (gemm_tiles.h). The list is compiled in
// KH_GEMM_TUNE_PARTS code objects: this file with -DKH_GEMM_TUNE_PART=p
// becomes gemm_tune<p>. Every candidate is correct for every shape and grid
// (tiles are grid-strided; tails are zero-filled or guarded).
#include "gemm_tiles.h"
#include "gemm_tune_list.h"

#ifndef KH_GEMM_TUNE_PART
#error "compile with -DKH_GEMM_TUNE_PART=<0 .. KH_GEMM_TUNE_PARTS-1>"
#endif

// A candidate's tile split assumes its own workgroup size (64 WGM WGN
// threads, one-dimensional); any other launch is refused (khg::refuse_launch).
#define KH_GEMM_TUNE_KERNEL(PART, MF, WGM, WGN, WTM, WTN, BK, PRIO, PIPE, SYM)                               \
  extern "C" __global__ void __launch_bounds__(64 * WGM * WGN) __attribute__((amdgpu_waves_per_eu(2)))         \
  SYM(KH_MEMREF2(const float, A), KH_MEMREF2(const float, B), KH_MEMREF2(float, C)) {                        \
    const uint32_t gxy = kh::group_size_word(), gz = kh::group_size_z_word();                                \
    KH_GEMM_ARGS_READY(gxy, gz);                                                                               \
    if (kh::threads_x_of(gxy) != 64 * WGM * WGN || kh::threads_y_of(gxy) != 1 || kh::threads_z_of(gz) != 1) { \
      khg::refuse_launch(KH_PTR(C), C_n0, C_n1, C_s0);                                                              \
      return;                                                                                                  \
    }                                                                                                          \
    khg::gemm_entry_pipe<WTM, WTN, BK, PRIO != 0, PIPE, WGM, WGN, MF>(KH_PTR(A), KH_PTR(B), KH_PTR(C), A_n0,  \
                                                                      B_n1, A_n1, A_s0, B_s0, C_s0);         \
  }

#if KH_GEMM_TUNE_PART == 0
KH_GEMM_TUNE_PART0(KH_GEMM_TUNE_KERNEL)
#elif KH_GEMM_TUNE_PART == 1
KH_GEMM_TUNE_PART1(KH_GEMM_TUNE_KERNEL)
#elif KH_GEMM_TUNE_PART == 2
KH_GEMM_TUNE_PART2(KH_GEMM_TUNE_KERNEL)
#elif KH_GEMM_TUNE_PART == 3
KH_GEMM_TUNE_PART3(KH_GEMM_TUNE_KERNEL)
#else
#error "KH_GEMM_TUNE_PART out of range"
#endif
static_assert(KH_GEMM_TUNE_PARTS == 4, "one #if branch per part");
