// Bench metrics: the formulas behind the bench's gflops_or_gbps column
// (bench/harness/metrics.cpp:5-52, pinned by test/unit/bench_metrics_test.cpp),
// in one place for the kernelh CLI's rows and comparators and for tests.
// Bytes are counted per launch as the reference counts them: every stream a
// kernel's argument list names, fused_gelu's dead `tmp` included (3 streams;
// the kernel itself moves 2), layernorm's gamma and beta once.
#include "kernelh/khrt_internal.hpp"

#include <initializer_list>
#include <cstring>
#include <string>

namespace {

double gflops_from_ms(double flops, double ms) { return flops * 1000.0 / ms / 1e9; }
double gbps_from_ms(double bytes, double ms) { return bytes * 1000.0 / ms / 1e9; }
double gemm_flops(double m, double n, double k) { return 2.0 * m * n * k; }
double gemm_bytes(double m, double n, double k) { return 4.0 * (m * k + k * n + m * n); }
double elementwise_bytes(double rows, double cols) { return 4.0 * 2.0 * rows * cols; }
double layernorm_bytes(double rows, double cols) { return elementwise_bytes(rows, cols) + 4.0 * 2.0 * cols; }
double scan_bytes(double n) { return 4.0 * 2.0 * n; }
double fused_gelu_bytes(double n) { return 4.0 * 3.0 * n; }
double attention_flops(double b, double h, double s, double d) { return 4.0 * b * h * s * s * d; }
double roofline_triad_bytes(double n) { return 4.0 * 3.0 * n; }
double roofline_fma_flops(double fmas) { return 2.0 * fmas; }

struct Formula {
  const char *name;
  int args;
  double (*f)(const double *);
};

const Formula kFormulas[] = {
    {"gflops_from_ms", 2, [](const double *a) { return gflops_from_ms(a[0], a[1]); }},
    {"gbps_from_ms", 2, [](const double *a) { return gbps_from_ms(a[0], a[1]); }},
    {"gemm_flops", 3, [](const double *a) { return gemm_flops(a[0], a[1], a[2]); }},
    {"gemm_bytes", 3, [](const double *a) { return gemm_bytes(a[0], a[1], a[2]); }},
    {"elementwise_bytes", 2, [](const double *a) { return elementwise_bytes(a[0], a[1]); }},
    {"layernorm_bytes", 2, [](const double *a) { return layernorm_bytes(a[0], a[1]); }},
    {"scan_bytes", 1, [](const double *a) { return scan_bytes(a[0]); }},
    {"fused_gelu_bytes", 1, [](const double *a) { return fused_gelu_bytes(a[0]); }},
    {"attention_flops", 4, [](const double *a) { return attention_flops(a[0], a[1], a[2], a[3]); }},
    {"roofline_triad_bytes", 1, [](const double *a) { return roofline_triad_bytes(a[0]); }},
    {"roofline_fma_flops", 1, [](const double *a) { return roofline_fma_flops(a[0]); }},
};

}  // namespace

extern "C" int khrt_bench_metric(const char *formula, const double *args, int nargs, double *out) {
  if (formula == nullptr || out == nullptr || (nargs > 0 && args == nullptr)) {
    return khrt::fail(KHRT_E_INVALID, "khrt_bench_metric: null argument");
  }
  for (const Formula &f : kFormulas) {
    if (std::strcmp(f.name, formula) != 0) continue;
    if (nargs != f.args) {
      return khrt::fail(KHRT_E_INVALID, std::string("khrt_bench_metric: ") + formula + " takes " +
                                            std::to_string(f.args) + " arguments, got " + std::to_string(nargs));
    }
    *out = f.f(args);
    return 0;
  }
  return khrt::fail(KHRT_E_INVALID, std::string("khrt_bench_metric: unknown formula '") + formula + "'");
}

extern "C" int khrt_bench_row_work(const char *kernel, const char *shape, double *work, int *is_flops) {
  if (kernel == nullptr || shape == nullptr || work == nullptr || is_flops == nullptr) {
    return khrt::fail(KHRT_E_INVALID, "khrt_bench_row_work: null argument");
  }
  kernelh::ShapeDims s;
  std::string why;
  if (!kernelh::parse_shape_text(shape, s, &why)) {
    return khrt::fail(KHRT_E_INVALID, "khrt_bench_row_work: malformed shape: expected " + why);
  }
  auto dim = [&](const char *key, int64_t dflt = -1) -> double {
    const auto it = s.find(key);
    return static_cast<double>(it == s.end() ? dflt : it->second);
  };
  auto need = [&](std::initializer_list<const char *> keys) {
    for (const char *k : keys)
      if (s.count(k) == 0) return false;
    return true;
  };
  const std::string k = kernel;
  *is_flops = 0;
  if ((k == "vecadd" || k == "roofline_triad") && need({"n"})) {
    *work = roofline_triad_bytes(dim("n"));  // two loads and a store of n floats
  } else if (k == "fused_gelu" && (need({"n"}) || need({"rows", "cols"}))) {
    *work = fused_gelu_bytes(s.count("n") ? dim("n") : dim("rows") * dim("cols"));
  } else if (k == "softmax" && need({"rows", "cols"})) {
    *work = elementwise_bytes(dim("rows"), dim("cols"));
  } else if (k == "layernorm" && need({"rows", "cols"})) {
    *work = layernorm_bytes(dim("rows"), dim("cols"));
  } else if (k == "scan" && need({"n"})) {
    *work = scan_bytes(dim("n"));
  } else if (k == "gemm" && need({"m", "n", "k"})) {
    *work = gemm_flops(dim("m"), dim("n"), dim("k"));
    *is_flops = 1;
  } else if (k == "attention" && need({"batch", "heads", "seq"})) {
    *work = attention_flops(dim("batch"), dim("heads"), dim("seq"), dim("head_dim", 64));
    *is_flops = 1;
  } else {
    return khrt::fail(KHRT_E_INVALID, "khrt_bench_row_work: no bench row for kernel '" + k + "' at shape '" +
                                          shape + "'");
  }
  return 0;
}
