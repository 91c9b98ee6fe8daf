// Comparator rows for `kernelh bench`: the hand-written HIP baselines
// (hipref-naive / hipref-vec, roofline_fma) from the code object embedded in
// the CLI, and rocBLAS and hipBLASLt fp32 GEMM as the vendor comparators.
//
// Mirrors the reference's bench backends (bench/harness/hipref_backend.cpp,
// rocblas_backend.cpp, roofline.cpp:100-145): same symbols, launch geometry
// and metric formulas, so results.csv rows are comparable.
#pragma once

#include <cstdint>
#include <functional>
#include <map>
#include <string>
#include <vector>

namespace khcli {

// Device buffers owned by one bench row, freed when it goes out of scope.
struct Bufs {
  std::vector<void *> ptrs;
  ~Bufs();
  // `count` floats filled with `fill` (nullptr on allocation failure).
  float *alloc(int64_t count, float fill);
};

// Each prepare_* allocates a row's buffers and returns its launcher; the
// caller counts the row's work with the shared bench formulas
// (khrt_bench_row_work).
// Prepares a hipref-naive / hipref-vec row (`variant` "naive" or "vec4").
bool prepare_hipref(const std::string &kernel, const std::string &variant,
                    const std::map<std::string, int64_t> &shape, Bufs &b, std::function<int()> &launch,
                    std::string &error);

// The vector-ALU FMA ceiling row (2^22 elements x 8192 FMAs); `fmas` is
// the FMA count of one launch.
bool prepare_roofline_fma(Bufs &b, std::function<int()> &launch, double &fmas, std::string &error);

// rocBLAS sgemm for a row-major m x k by k x n product (dlopen'ed; an
// error, not a crash, when librocblas is absent).
bool prepare_rocblas_gemm(const std::map<std::string, int64_t> &shape, Bufs &b, std::function<int()> &launch,
                          std::string &error);

// hipBLASLt fp32 GEMM (hipblasLtMatmul with the heuristic's first algorithm
// and up to 64 MiB of workspace), the same product and layout as the
// rocBLAS row; dlopen'ed, an error when absent or without an fp32 algorithm.
bool prepare_hipblaslt_gemm(const std::map<std::string, int64_t> &shape, Bufs &b, std::function<int()> &launch,
                            std::string &error);

}  // namespace khcli
