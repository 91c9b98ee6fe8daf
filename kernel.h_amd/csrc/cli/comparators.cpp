// Comparator rows for `kernelh bench` (see comparators.hpp).
#include "comparators.hpp"

#include "khrt.h"

#include <dlfcn.h>
#include <hipblaslt/hipblaslt.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cstring>
#include <memory>

// The hipref code object, embedded by build.py (gen/kh_cli_embed.S).
extern "C" const unsigned char kh_cli_co_hipref[];
extern "C" const unsigned char kh_cli_co_hipref_end[];

namespace khcli {

Bufs::~Bufs() {
  for (void *p : ptrs)
    if (p) khrt_free(p);
}

// A failed allocation is recorded as nullptr so callers can check `ptrs`.
float *Bufs::alloc(int64_t count, float fill) {
  void *p = nullptr;
  if (khrt_malloc(&p, static_cast<size_t>(std::max<int64_t>(count, 1)) * 4) != 0) {
    ptrs.push_back(nullptr);
    return nullptr;
  }
  ptrs.push_back(p);
  khrt_fill_f32(p, fill, static_cast<size_t>(count), nullptr);
  return static_cast<float *>(p);
}

namespace {

int64_t get(const std::map<std::string, int64_t> &s, const char *k, int64_t dflt = 0) {
  auto it = s.find(k);
  return it == s.end() ? dflt : it->second;
}

// Raw kernel arguments: each value in its own 8-byte slot, addressed by the
// params array hipModuleLaunchKernel takes.
struct RawArgs {
  std::vector<uint64_t> slots;
  std::vector<void *> ptrs;
  template <class T>
  RawArgs &add(T v) {
    static_assert(sizeof(T) <= 8, "slot size");
    uint64_t s = 0;
    std::memcpy(&s, &v, sizeof(T));
    slots.push_back(s);
    return *this;
  }
  void **params() {
    ptrs.clear();
    for (auto &s : slots) ptrs.push_back(&s);
    return ptrs.data();
  }
};

// Module of the embedded comparators, loaded on first use and kept for the
// process lifetime.
bool hipref_function(const char *symbol, void **fn, std::string &error) {
  static void *module = nullptr;
  if (module == nullptr) {
    const size_t size = static_cast<size_t>(kh_cli_co_hipref_end - kh_cli_co_hipref);
    if (size == 0) {
      error = "hipref code object not embedded in this build";
      return false;
    }
    if (khrt_module_load_data(&module, kh_cli_co_hipref, size) != 0) {
      error = std::string("hipref code object failed to load: ") + khrt_last_error();
      module = nullptr;
      return false;
    }
  }
  if (khrt_module_get_function(fn, module, symbol) != 0) {
    error = std::string("hipref symbol '") + symbol + "': " + khrt_last_error();
    return false;
  }
  return true;
}

khrt_dim3 dim(int64_t x, int64_t y = 1) {
  return khrt_dim3{static_cast<unsigned>(x), static_cast<unsigned>(y), 1};
}

std::function<int()> raw_launcher(void *fn, khrt_dim3 grid, khrt_dim3 block, std::shared_ptr<RawArgs> args) {
  return [=] { return khrt_launch_raw(fn, grid, block, 0, nullptr, args->params()); };
}

}  // namespace

bool prepare_hipref(const std::string &kernel, const std::string &variant,
                    const std::map<std::string, int64_t> &s, Bufs &b, std::function<int()> &launch,
                    std::string &error) {
  const bool vec = variant == "vec4";
  void *fn = nullptr;
  if (kernel == "softmax" || kernel == "layernorm") {
    const int64_t r = get(s, "rows"), c = get(s, "cols");
    if (vec && c % 4 != 0) {
      error = kernel + " hipref-vec needs cols % 4 == 0";
      return false;
    }
    if (!hipref_function((kernel + "_" + variant).c_str(), &fn, error)) return false;
    float *x = b.alloc(r * c, 0.5f), *y = b.alloc(r * c, 0.0f);
    auto args = std::make_shared<RawArgs>();
    if (kernel == "softmax") {
      args->add(x).add(y).add(static_cast<int>(r)).add(static_cast<int>(c));
      const int64_t block = std::min<int64_t>((std::min<int64_t>(c, 256) + 63) / 64 * 64, 256);
      launch = raw_launcher(fn, dim(r), dim(block), args);
    } else {
      float *g = b.alloc(c, 1.0f), *bt = b.alloc(c, 0.0f);
      args->add(x).add(g).add(bt).add(y).add(static_cast<int>(r)).add(static_cast<int>(c));
      launch = raw_launcher(fn, dim(r), dim(256), args);
    }
  } else if (kernel == "fused_gelu") {
    const int64_t n = get(s, "n");
    if (vec && n % 4 != 0) {
      error = "fused_gelu hipref-vec needs n % 4 == 0";
      return false;
    }
    if (!hipref_function(("fused_gelu_" + variant).c_str(), &fn, error)) return false;
    float *x = b.alloc(n, 0.25f), *y = b.alloc(n, 0.0f);
    auto args = std::make_shared<RawArgs>();
    args->add(x).add(y).add(static_cast<int>(n));
    launch = raw_launcher(fn, dim((n + 255) / 256), dim(256), args);
  } else if (kernel == "scan") {
    const int64_t n = get(s, "n"), t = (n + 255) / 256;
    void *fn2 = nullptr;
    if (!hipref_function(("scan_pass1_" + variant).c_str(), &fn, error) ||
        !hipref_function(("scan_totals_" + variant).c_str(), &fn2, error)) {
      return false;
    }
    float *x = b.alloc(n, 0.5f), *y = b.alloc(n, 0.0f), *tot = b.alloc(t, 0.0f);
    auto a1 = std::make_shared<RawArgs>(), a2 = std::make_shared<RawArgs>();
    a1->add(x).add(y).add(tot).add(static_cast<int>(n)).add(static_cast<int>(t));
    a2->add(tot).add(y).add(static_cast<int>(t)).add(static_cast<int>(n));
    // Both passes form one measurement (hipref_backend.cpp:58-75).
    launch = [=] {
      if (int rc = khrt_launch_raw(fn, dim(t), dim(256), 0, nullptr, a1->params())) return rc;
      return khrt_launch_raw(fn2, dim(1), dim(256), 0, nullptr, a2->params());
    };
  } else if (kernel == "gemm") {
    if (vec) {
      error = "gemm has no hipref-vec variant (only the naive tiled comparator)";
      return false;
    }
    const int64_t m = get(s, "m"), n = get(s, "n"), k = get(s, "k");
    if (!hipref_function("gemm_tiled", &fn, error)) return false;
    float *A = b.alloc(m * k, 1.0f), *B = b.alloc(k * n, 1.0f), *C = b.alloc(m * n, 0.0f);
    auto args = std::make_shared<RawArgs>();
    args->add(A).add(B).add(C).add(static_cast<int>(m)).add(static_cast<int>(n)).add(static_cast<int>(k));
    launch = raw_launcher(fn, dim((n + 31) / 32, (m + 31) / 32), khrt_dim3{32, 8, 1}, args);
  } else {
    error = "hipref backend has no comparator for kernel '" + kernel + "'";
    return false;
  }
  for (void *p : b.ptrs) {
    if (p == nullptr) {
      error = "comparator buffer allocation failed";
      return false;
    }
  }
  return true;
}

bool prepare_roofline_fma(Bufs &b, std::function<int()> &launch, double &fmas, std::string &error) {
  constexpr int64_t kElems = 1 << 22;
  constexpr int kIters = 8192;
  void *fn = nullptr;
  if (!hipref_function("roofline_fma", &fn, error)) return false;
  float *c = b.alloc(kElems, 1.0f);
  if (c == nullptr) {
    error = "buffer allocation failed";
    return false;
  }
  auto args = std::make_shared<RawArgs>();
  args->add(c).add(static_cast<int>(kElems)).add(kIters);
  launch = raw_launcher(fn, dim((kElems + 255) / 256), dim(256), args);
  fmas = static_cast<double>(kElems) * kIters;
  return true;
}

namespace {

struct Rocblas {
  using create_t = rocblas_status (*)(rocblas_handle *);
  using sgemm_t = rocblas_status (*)(rocblas_handle, rocblas_operation, rocblas_operation, rocblas_int, rocblas_int,
                                     rocblas_int, const float *, const float *, rocblas_int, const float *,
                                     rocblas_int, const float *, float *, rocblas_int);
  void *lib = nullptr;
  create_t create = nullptr;
  sgemm_t sgemm = nullptr;
  rocblas_handle handle = nullptr;
  std::string error;

  Rocblas() {
    for (const char *name : {"librocblas.so.5", "librocblas.so", "/opt/rocm/lib/librocblas.so"}) {
      lib = dlopen(name, RTLD_NOW | RTLD_LOCAL);
      if (lib) break;
    }
    if (!lib) {
      error = "librocblas not found";
      return;
    }
    create = reinterpret_cast<create_t>(dlsym(lib, "rocblas_create_handle"));
    sgemm = reinterpret_cast<sgemm_t>(dlsym(lib, "rocblas_sgemm"));
    if (!create || !sgemm) {
      error = "librocblas lacks rocblas_create_handle / rocblas_sgemm";
      return;
    }
    if (create(&handle) != rocblas_status_success) error = "rocblas_create_handle failed";
  }
};

Rocblas &rocblas() {
  // One handle for the process (the handle outlives every row; the library
  // stays loaded until exit).
  static Rocblas r;
  return r;
}

}  // namespace

bool prepare_rocblas_gemm(const std::map<std::string, int64_t> &s, Bufs &b, std::function<int()> &launch,
                          std::string &error) {
  Rocblas &r = rocblas();
  if (!r.error.empty()) {
    error = r.error;
    return false;
  }
  const int64_t m = get(s, "m"), n = get(s, "n"), k = get(s, "k");
  float *A = b.alloc(m * k, 1.0f), *B = b.alloc(k * n, 1.0f), *C = b.alloc(m * n, 0.0f);
  if (!A || !B || !C) {
    error = "rocblas buffer allocation failed";
    return false;
  }
  // Row-major C = A B is column-major C^T = B^T A^T: B (n x k, ld n) times
  // A (k x m, ld k) into C (n x m, ld n).
  launch = [=, &r] {
    const float one = 1.0f, zero = 0.0f;
    const rocblas_status st = r.sgemm(r.handle, rocblas_operation_none, rocblas_operation_none,
                                      static_cast<rocblas_int>(n), static_cast<rocblas_int>(m),
                                      static_cast<rocblas_int>(k), &one, B, static_cast<rocblas_int>(n), A,
                                      static_cast<rocblas_int>(k), &zero, C, static_cast<rocblas_int>(n));
    return st == rocblas_status_success ? 0 : 1;
  };
  return true;
}

namespace {

// hipBLASLt through its C API, dlopen'ed like rocBLAS: one handle, and per
// shape one matmul description, three column-major layouts, the heuristic's
// first algorithm and its workspace (kept for the process lifetime, a few
// shapes per run).
struct Hipblaslt {
  using create_t = hipblasStatus_t (*)(hipblasLtHandle_t *);
  using desc_create_t = hipblasStatus_t (*)(hipblasLtMatmulDesc_t *, hipblasComputeType_t, hipDataType);
  using layout_create_t = hipblasStatus_t (*)(hipblasLtMatrixLayout_t *, hipDataType, uint64_t, uint64_t, int64_t);
  using pref_create_t = hipblasStatus_t (*)(hipblasLtMatmulPreference_t *);
  using pref_set_t = hipblasStatus_t (*)(hipblasLtMatmulPreference_t, hipblasLtMatmulPreferenceAttributes_t,
                                         const void *, size_t);
  using heuristic_t = hipblasStatus_t (*)(hipblasLtHandle_t, hipblasLtMatmulDesc_t, hipblasLtMatrixLayout_t,
                                          hipblasLtMatrixLayout_t, hipblasLtMatrixLayout_t, hipblasLtMatrixLayout_t,
                                          hipblasLtMatmulPreference_t, int, hipblasLtMatmulHeuristicResult_t[],
                                          int *);
  using matmul_t = hipblasStatus_t (*)(hipblasLtHandle_t, hipblasLtMatmulDesc_t, const void *, const void *,
                                       hipblasLtMatrixLayout_t, const void *, hipblasLtMatrixLayout_t, const void *,
                                       const void *, hipblasLtMatrixLayout_t, void *, hipblasLtMatrixLayout_t,
                                       const hipblasLtMatmulAlgo_t *, void *, size_t, hipStream_t);
  void *lib = nullptr;
  create_t create = nullptr;
  desc_create_t desc_create = nullptr;
  layout_create_t layout_create = nullptr;
  pref_create_t pref_create = nullptr;
  pref_set_t pref_set = nullptr;
  heuristic_t heuristic = nullptr;
  matmul_t matmul = nullptr;
  hipblasLtHandle_t handle = nullptr;
  std::string error;

  template <class F>
  bool sym(F &f, const char *name) {
    f = reinterpret_cast<F>(dlsym(lib, name));
    if (!f) error = std::string("libhipblaslt lacks ") + name;
    return f != nullptr;
  }

  Hipblaslt() {
    for (const char *name : {"libhipblaslt.so.1", "libhipblaslt.so", "/opt/rocm/lib/libhipblaslt.so"}) {
      lib = dlopen(name, RTLD_NOW | RTLD_LOCAL);
      if (lib) break;
    }
    if (!lib) {
      error = "libhipblaslt not found";
      return;
    }
    if (!sym(create, "hipblasLtCreate") || !sym(desc_create, "hipblasLtMatmulDescCreate") ||
        !sym(layout_create, "hipblasLtMatrixLayoutCreate") || !sym(pref_create, "hipblasLtMatmulPreferenceCreate") ||
        !sym(pref_set, "hipblasLtMatmulPreferenceSetAttribute") ||
        !sym(heuristic, "hipblasLtMatmulAlgoGetHeuristic") || !sym(matmul, "hipblasLtMatmul")) {
      return;
    }
    if (create(&handle) != HIPBLAS_STATUS_SUCCESS) error = "hipblasLtCreate failed";
  }
};

Hipblaslt &hipblaslt() {
  static Hipblaslt h;
  return h;
}

}  // namespace

bool prepare_hipblaslt_gemm(const std::map<std::string, int64_t> &s, Bufs &b, std::function<int()> &launch,
                            std::string &error) {
  Hipblaslt &h = hipblaslt();
  if (!h.error.empty()) {
    error = h.error;
    return false;
  }
  const int64_t m = get(s, "m"), n = get(s, "n"), k = get(s, "k");
  float *A = b.alloc(m * k, 1.0f), *B = b.alloc(k * n, 1.0f), *C = b.alloc(m * n, 0.0f);
  if (!A || !B || !C) {
    error = "hipblaslt buffer allocation failed";
    return false;
  }
  // Row-major C = A B as column-major C^T (n x m) = B^T (n x k) A^T (k x m),
  // fp32 data, fp32 compute, no transposes.
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t lx = nullptr, ly = nullptr, lc = nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (h.desc_create(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS ||
      h.layout_create(&lx, HIP_R_32F, n, k, n) != HIPBLAS_STATUS_SUCCESS ||
      h.layout_create(&ly, HIP_R_32F, k, m, k) != HIPBLAS_STATUS_SUCCESS ||
      h.layout_create(&lc, HIP_R_32F, n, m, n) != HIPBLAS_STATUS_SUCCESS ||
      h.pref_create(&pref) != HIPBLAS_STATUS_SUCCESS) {
    error = "hipblaslt descriptor creation failed";
    return false;
  }
  const uint64_t ws_bytes = 64ull << 20;
  h.pref_set(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws_bytes, sizeof ws_bytes);
  auto result = std::make_shared<hipblasLtMatmulHeuristicResult_t>();
  int found = 0;
  if (h.heuristic(h.handle, desc, lx, ly, lc, lc, pref, 1, result.get(), &found) != HIPBLAS_STATUS_SUCCESS ||
      found < 1) {
    error = "hipblaslt has no fp32 algorithm for this shape";
    return false;
  }
  float *ws = result->workspaceSize > 0 ? b.alloc(static_cast<int64_t>((result->workspaceSize + 3) / 4), 0.0f) : nullptr;
  if (result->workspaceSize > 0 && ws == nullptr) {
    error = "hipblaslt workspace allocation failed";
    return false;
  }
  launch = [=, &h] {
    const float one = 1.0f, zero = 0.0f;
    const hipblasStatus_t st = h.matmul(h.handle, desc, &one, B, lx, A, ly, &zero, C, lc, C, lc, &result->algo, ws,
                                        result->workspaceSize, nullptr);
    return st == HIPBLAS_STATUS_SUCCESS ? 0 : 1;
  };
  return true;
}

}  // namespace khcli
