// kernelh - command-line driver for the gfx950 kernel.h templates.
//
// The reference's CLI surface for this path (tools/kernelh/main.cpp):
//   kernelh compile --kernel <name> --shape k=v,... --target <t> --out <dir>
//                   [--resources]                          (main.cpp:435-646)
//   kernelh tune    --kernel gemm --shape m=..,n=..,k=.. --out <dir> [...]
//                                                          (main.cpp:649-1420)
//   kernelh bench   --suite <roofline|kernelh|rocblas|hipblaslt|hipref|all> --out <path>
//                   [--occupancy] [--kernel <name> --shape ... [--backend <b>]]
//   kernelh bench   --occupancy --kernel <name> --target amdgcn-gfx950
//                   [--shape ...] [--threads N] --out <dir>   (occupancy only)
//                                                          (main.cpp:2154-2228,
//                                                   run_bench.cpp:111-127)
// Exit codes as in the reference (main.cpp:125-127, run_bench.hpp:9-10):
// 0 ok, 1 operational failure, 2 usage error, 77 skipped (no GPU).
//
// compile writes <name>.hsaco (the embedded bare-ELF gfx950 code object whose
// extern "C" symbol is <name>), <name>.isa (its disassembly, when the ROCm
// llvm-objdump is installed) and, with --resources, resources.json. Shapes
// are validated against the template (the launcher geometry must resolve);
// the code objects read sizes from the memref descriptors at run time, so
// one object serves every shape.
//
// bench backends (bench/harness/run_bench.cpp:48-66): kernelh (the gfx950
// templates), rocblas and hipblaslt (vendor fp32 GEMM), hipref-naive / hipref-vec
// (hand-written HIP comparators embedded in this executable) and roofline
// (triad bandwidth, vector FMA ceiling).
// bench times each row with the reference's method: 5 warmup launches, then
// the median of 20 event-timed launches (bench/harness/timer.cpp:29-67), and
// writes the G32 results.csv schema
// kernel,shape,backend,ms_median,gflops_or_gbps,timestamp,device
// (bench/harness/csv.cpp:9-10).
#include "khrt.h"

#include "args.hpp"
#include "comparators.hpp"
#include "kernelh/shape_text.hpp"
#include "tune.hpp"

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <filesystem>
#include <fstream>
#include <functional>
#include <iostream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

namespace fs = std::filesystem;

namespace {

constexpr int kExitOk = 0;
constexpr int kExitOperational = 1;
constexpr int kExitUsage = 2;
constexpr int kExitSkip = 77;

void usage(std::ostream &os) {
  os << "kernelh - kernel.h templates on AMD Instinct MI355X (gfx950)\n\n"
     << "usage: kernelh <compile|bench|tune|info> [options]\n\n"
     << "compile options:\n"
     << "  --kernel <name>       template: vecadd, gemm, softmax, layernorm, scan,\n"
     << "                        scan_totals, fused_gelu, attention\n"
     << "  --shape k=v,k=v,...   problem dims (e.g. n=1024; rows=..,cols=..;\n"
     << "                        m=..,n=..,k=..; batch=..,heads=..,seq=..,head_dim=64)\n"
     << "  --target <t>          amdgcn-gfx950 (default; the only code-object target)\n"
     << "  --out <dir>           write <dir>/<kernel>.{hsaco,isa} (created if missing)\n"
     << "  --resources           also write <dir>/resources.json\n\n"
     << "tune options (GEMM only): kernelh tune --help\n"
     << "  --shape m=..,n=..,k=.. --out <dir> [--max-candidates n] [--sample n]\n"
     << "  [--refine-budget n] [--timeout s] [--cache path]; writes <dir>/tune-results.csv,\n"
     << "  prints the best config\n\n"
     << "bench options:\n"
     << "  --suite <name>        roofline, kernelh, rocblas, hipblaslt, hipref, all (default: all)\n"
     << "  --backend <name>      with --kernel: kernelh (default), rocblas, hipblaslt,\n"
     << "                        hipref-naive, hipref-vec, roofline\n"
     << "  --kernel <name>       single-row mode: time one template ...\n"
     << "  --shape k=v,...       ... at this shape\n"
     << "  --out <path>          results.csv path or directory (required)\n"
     << "  --warmup <n>          warmup launches (default 5)\n"
     << "  --iters <n>           timed launches, median reported (default 20)\n"
     << "  --occupancy           write occupancy.{json,md} next to results.csv\n"
     << "occupancy-only mode (times nothing, needs no device):\n"
     << "  kernelh bench --occupancy --kernel <name> --target amdgcn-gfx950\n"
     << "                [--shape k=v,...] [--threads N] --out <dir>\n"
     << "  writes <dir>/occupancy.{json,md} for the symbol the launcher runs at that\n"
     << "  shape (default shapes as the reference's); --threads (1..1048576) overrides\n"
     << "  the launcher's workgroup size\n\n"
     << "info                    print the live device and the gfx950 limits entry\n\n"
     << "--help prints this usage and exits 0.\n";
}

std::string json_escape(const std::string &s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    if (static_cast<unsigned char>(c) < 0x20) continue;
    o += c;
  }
  return o;
}

std::string exe_dir() {
  std::error_code ec;
  const fs::path p = fs::read_symlink("/proc/self/exe", ec);
  return ec ? std::string(".") : p.parent_path().string();
}

const char *code_object_of(const std::string &kernel) { return kernel == "scan_totals" ? "scan" : kernel.c_str(); }

// resources.json: the reference's keys (kernel, target, vgpr_count,
// sgpr_count, lds_bytes, wavefront_size, occupancy_estimate;
// resource_reporter.hpp:50-58) plus this build's extras. occupancy_estimate
// is the reference's register-limited waves per CU,
// floor(reg_file_per_cu / (registers x wavefront_size)) clamped to
// [1, waves_per_cu] (resource_reporter.cpp:232-255), where registers counts
// the VGPRs and AGPRs that share gfx950's register file.
std::string resources_json(const std::string &kernel, const std::string &shape) {
  // Resources of the symbol the launcher runs at this shape (a template may
  // carry variants, e.g. gemm_small_pf2 or softmax_wide).
  char sym[64] = {0};
  if (khrt_template_launch_symbol(kernel.c_str(), shape.c_str(), sym, sizeof(sym)) != 0) return "";
  khrt_kernel_resources r{};
  if (khrt_template_resources(sym, &r) != 0) return "";
  khrt_dim3 grid{}, block{};
  khrt_template_geometry(kernel.c_str(), shape.c_str(), &grid, &block);
  khrt_device_limits lim{};
  khrt_device_limits_for("gfx950", &lim);
  khrt_occupancy_input in{kernel.c_str(), "gfx950", shape.c_str(), r.vgpr_count + r.agpr_count, r.lds_bytes,
                          static_cast<int32_t>(block.x * block.y * block.z)};
  khrt_occupancy_report rep{};
  khrt_compute_occupancy(&in, &lim, nullptr, &rep);
  std::ostringstream os;
  os << "{\n  \"kernel\": \"" << json_escape(kernel) << "\",\n  \"symbol\": \"" << json_escape(sym)
     << "\",\n  \"target\": \"amdgcn-gfx950\",\n"
     << "  \"shape\": \"" << json_escape(shape) << "\",\n"
     << "  \"vgpr_count\": " << r.vgpr_count << ",\n  \"agpr_count\": " << r.agpr_count << ",\n"
     << "  \"sgpr_count\": " << r.sgpr_count << ",\n  \"lds_bytes\": " << r.lds_bytes << ",\n"
     << "  \"scratch_bytes\": " << r.private_segment_bytes << ",\n  \"wavefront_size\": " << r.wavefront_size
     << ",\n  \"occupancy_estimate\": " << rep.vgpr_limited_waves
     << ",\n  \"max_flat_workgroup_size\": " << r.max_flat_workgroup_size << ",\n"
     << "  \"launch\": {\"grid\": [" << grid.x << ", " << grid.y << ", " << grid.z << "], \"block\": [" << block.x
     << ", " << block.y << ", " << block.z << "]},\n"
     << "  \"theoretical_occupancy_pct\": " << rep.theoretical_pct << "\n}\n";
  return os.str();
}

int run_compile(int argc, char **argv) {
  std::string kernel, shape, target = "amdgcn-gfx950", out;
  bool resources = false;
  for (khcli::ArgCursor a(argc, argv, 2); !a.done();) {
    if (a.flag("--help") || a.flag("-h")) {
      usage(std::cout);
      return kExitOk;
    }
    if (a.value("--kernel", kernel) || a.value("--shape", shape) || a.value("--target", target) ||
        a.value("--out", out)) {
      continue;
    }
    if (a.flag("--resources")) {
      resources = true;
      continue;
    }
    std::cerr << "error: unknown compile option '" << a.word() << "'\n";
    usage(std::cerr);
    return kExitUsage;
  }
  if (kernel.empty() || shape.empty() || out.empty()) {
    std::cerr << "error: compile needs --kernel, --shape and --out\n";
    usage(std::cerr);
    return kExitUsage;
  }
  kernelh::ShapeDims parsed;
  std::string why;
  if (!kernelh::parse_shape_text(shape, parsed, &why)) {
    std::cerr << "error: malformed --shape: expected " << why << "\n";
    return kExitUsage;
  }
  const std::string token = target.rfind("amdgcn-", 0) == 0 ? target.substr(7) : target;
  khrt_device_limits lim{};
  if (khrt_device_limits_for(token.c_str(), &lim) != 0) {
    std::cerr << "error: " << khrt_last_error() << "\n"
              << "error: valid --target values: amdgcn-gfx950\n";
    return kExitOperational;
  }
  if (token != "gfx950") {
    std::cerr << "error: this build emits gfx950 code objects only (asked for " << target << ")\n"
              << "error: valid --target values: amdgcn-gfx950\n";
    return kExitOperational;
  }
  const void *image = nullptr;
  size_t size = 0;
  if (khrt_template_code_object(kernel.c_str(), &image, &size) != 0) {
    std::cerr << "error: " << khrt_last_error() << "\n";
    return kExitOperational;
  }
  khrt_dim3 grid{}, block{};
  if (khrt_template_geometry(kernel.c_str(), shape.c_str(), &grid, &block) != 0) {
    std::cerr << "error: " << khrt_last_error() << "\n";
    return kExitOperational;
  }
  std::error_code ec;
  fs::create_directories(out, ec);
  const fs::path hsaco = fs::path(out) / (kernel + ".hsaco");
  {
    std::ofstream f(hsaco, std::ios::binary);
    f.write(static_cast<const char *>(image), static_cast<std::streamsize>(size));
    if (!f) {
      std::cerr << "error: cannot write " << hsaco << "\n";
      return kExitOperational;
    }
  }
  std::cout << "wrote " << hsaco.string() << "\n";
  // The disassembly of the build's own code object, when available.
  const fs::path isa = fs::path(out) / (kernel + ".isa");
  const fs::path prebuilt = fs::path(exe_dir()) / "co" / (std::string(code_object_of(kernel)) + ".isa");
  if (fs::exists(prebuilt)) {
    fs::copy_file(prebuilt, isa, fs::copy_options::overwrite_existing, ec);
    if (!ec) std::cout << "wrote " << isa.string() << "\n";
  }
  if (resources) {
    const fs::path rj = fs::path(out) / "resources.json";
    std::ofstream f(rj);
    f << resources_json(kernel, shape);
    std::cout << "wrote " << rj.string() << "\n";
  }
  std::cout << "launch grid (" << grid.x << "," << grid.y << "," << grid.z << ") block (" << block.x << ","
            << block.y << "," << block.z << ")\n";
  std::cout << "compile ok\n";
  return kExitOk;
}

// ---------------------------------------------------------------- bench

struct Row {
  std::string kernel, shape;
  std::string backend = "kernelh";  // kernelh, rocblas, hipblaslt, hipref-naive, hipref-vec, roofline
};

using khcli::Bufs;

int64_t get(const std::map<std::string, int64_t> &s, const char *k, int64_t dflt = 0) {
  auto it = s.find(k);
  return it == s.end() ? dflt : it->second;
}

// Allocates a kernelh row's buffers and returns its launcher closure.
bool prepare_kernelh(const std::string &k, const kernelh::ShapeDims &s, Bufs &b, std::function<int()> &launch,
                     std::string &error) {
  error = "unknown kernel or allocation failure";
  if (k == "vecadd") {
    const int64_t n = get(s, "n");
    float *a = b.alloc(n, 1.0f), *bb = b.alloc(n, 2.0f), *c = b.alloc(n, 0.0f);
    launch = [=] { return kh_vecadd(a, bb, c, n, nullptr); };
  } else if (k == "fused_gelu") {
    const int64_t n = s.count("n") ? get(s, "n") : get(s, "rows") * get(s, "cols");
    float *x = b.alloc(n, 0.25f), *o = b.alloc(n, 0.0f);
    launch = [=] { return kh_fused_gelu(x, nullptr, o, n, nullptr); };
  } else if (k == "softmax" || k == "layernorm") {
    const int64_t r = get(s, "rows"), c = get(s, "cols");
    float *x = b.alloc(r * c, 0.5f), *y = b.alloc(r * c, 0.0f);
    if (k == "softmax") {
      launch = [=] { return kh_softmax(x, y, r, c, nullptr); };
    } else {
      float *g = b.alloc(c, 1.0f), *bt = b.alloc(c, 0.0f);
      launch = [=] { return kh_layernorm(x, g, bt, y, r, c, nullptr); };
    }
  } else if (k == "scan") {
    const int64_t n = get(s, "n"), T = (n + 255) / 256;
    float *x = b.alloc(n, 0.5f), *y = b.alloc(n, 0.0f), *th = b.alloc(T, 0.0f), *tl = b.alloc(T, 0.0f);
    launch = [=] { return kh_scan(x, y, nullptr, th, tl, n, nullptr); };
  } else if (k == "gemm") {
    const int64_t m = get(s, "m"), n = get(s, "n"), kk = get(s, "k");
    float *A = b.alloc(m * kk, 1.0f), *B = b.alloc(kk * n, 1.0f), *C = b.alloc(m * n, 0.0f);
    launch = [=] { return kh_gemm(A, B, C, m, n, kk, nullptr); };
  } else if (k == "attention") {
    const int64_t bt = get(s, "batch"), h = get(s, "heads"), sq = get(s, "seq"), d = get(s, "head_dim", 64);
    const int64_t e = bt * h * sq * d;
    float *Q = b.alloc(e, 0.01f), *K = b.alloc(e, 0.02f), *V = b.alloc(e, 1.0f), *O = b.alloc(e, 0.0f);
    launch = [=] { return kh_attention(Q, K, V, O, bt, h, sq, d, nullptr); };
  } else if (k == "roofline_triad") {
    const int64_t n = get(s, "n");
    float *a = b.alloc(n, 1.0f), *bb = b.alloc(n, 2.0f), *c = b.alloc(n, 0.0f);
    launch = [=] { return kh_roofline_triad(a, bb, c, n, nullptr); };
  } else {
    return false;
  }
  for (void *p : b.ptrs)
    if (p == nullptr) return false;
  return true;
}

// Prepares any row and counts its work with the reference's formulas
// (bench/harness/metrics.cpp, through khrt_bench_row_work), so rows compare
// across backends: bytes for the bandwidth kernels, 2mnk / 4bhs^2d FLOPs.
bool prepare(const Row &row, Bufs &b, std::function<int()> &launch, double &work, bool &flops, std::string &error) {
  kernelh::ShapeDims s;
  std::string why;
  if (!kernelh::parse_shape_text(row.shape, s, &why)) {
    error = "malformed shape: expected " + why;
    return false;
  }
  const std::string &k = row.kernel;
  if ((row.backend == "rocblas" || row.backend == "hipblaslt") && k != "gemm") {
    error = row.backend + " backend only benchmarks gemm (got '" + k + "')";
    return false;
  }
  if (k == "roofline_fma") {
    double fmas = 0.0;
    flops = true;
    return khcli::prepare_roofline_fma(b, launch, fmas, error) &&
           khrt_bench_metric("roofline_fma_flops", &fmas, 1, &work) == 0;
  }
  const bool ok = row.backend == "hipref-naive" || row.backend == "hipref-vec"
                      ? khcli::prepare_hipref(k, row.backend == "hipref-vec" ? "vec4" : "naive", s, b, launch, error)
                  : row.backend == "rocblas"   ? khcli::prepare_rocblas_gemm(s, b, launch, error)
                  : row.backend == "hipblaslt" ? khcli::prepare_hipblaslt_gemm(s, b, launch, error)
                                               : prepare_kernelh(k, s, b, launch, error);
  if (!ok) return false;
  int is_flops = 0;
  if (khrt_bench_row_work(k.c_str(), row.shape.c_str(), &work, &is_flops) != 0) {
    error = khrt_last_error();
    return false;
  }
  flops = is_flops != 0;
  return true;
}

// Warmup, then the median of `iters` event-timed launches (timer.cpp:29-67).
bool time_row(const std::function<int()> &launch, int warmup, int iters, double &ms_median) {
  for (int i = 0; i < warmup; ++i)
    if (launch() != 0) return false;
  if (khrt_device_synchronize() != 0) return false;
  void *e0 = nullptr, *e1 = nullptr;
  khrt_event_create(&e0);
  khrt_event_create(&e1);
  std::vector<double> ms;
  for (int i = 0; i < iters; ++i) {
    khrt_event_record(e0, nullptr);
    if (launch() != 0) return false;
    khrt_event_record(e1, nullptr);
    khrt_event_synchronize(e1);
    float t = 0.0f;
    khrt_event_elapsed_ms(&t, e0, e1);
    ms.push_back(t);
  }
  khrt_event_destroy(e0);
  khrt_event_destroy(e1);
  std::sort(ms.begin(), ms.end());
  ms_median = ms.size() % 2 ? ms[ms.size() / 2] : 0.5 * (ms[ms.size() / 2 - 1] + ms[ms.size() / 2]);
  return true;
}

std::string now_iso() {
  const std::time_t t = std::time(nullptr);
  char buf[32];
  std::strftime(buf, sizeof(buf), "%Y-%m-%dT%H:%M:%SZ", std::gmtime(&t));
  return buf;
}

// Suites as in the reference (bench/harness/suites.cpp:22-101), with the
// BASELINE configurations added to the kernelh suite.
std::vector<Row> gemm_rows(const std::string &backend) {
  std::vector<Row> rows;
  for (const int64_t n : {512, 1024, 2048, 4096, 8192}) {
    const std::string d = std::to_string(n);
    rows.push_back({"gemm", "m=" + d + ",n=" + d + ",k=" + d, backend});
  }
  return rows;
}

std::vector<Row> kernelh_rows() {
  std::vector<Row> rows = gemm_rows("kernelh");
  rows.push_back({"gemm", "m=8192,n=8192,k=256"});
  rows.push_back({"vecadd", "n=16777216"});
  for (const char *shape : {"rows=4096,cols=1024", "rows=16384,cols=4096"}) {
    rows.push_back({"softmax", shape});
    rows.push_back({"layernorm", shape});
  }
  for (const char *n : {"n=100000", "n=1000000", "n=67108864"}) rows.push_back({"scan", n});
  for (const char *n : {"n=1048576", "n=4194304", "n=67108864"}) rows.push_back({"fused_gelu", n});
  for (const char *shape : {"batch=2,heads=8,seq=512,head_dim=64", "batch=2,heads=8,seq=1024,head_dim=64",
                            "batch=4,heads=16,seq=1024,head_dim=64", "batch=4,heads=16,seq=4096,head_dim=64"})
    rows.push_back({"attention", shape});
  return rows;
}

std::vector<Row> hipref_rows() {
  std::vector<Row> rows;
  for (const char *shape : {"rows=4096,cols=1024", "rows=16384,cols=4096"}) {
    for (const char *k : {"softmax", "layernorm"}) {
      rows.push_back({k, shape, "hipref-naive"});
      rows.push_back({k, shape, "hipref-vec"});
    }
  }
  for (const char *n : {"n=100000", "n=1000000"}) {
    rows.push_back({"scan", n, "hipref-naive"});
    rows.push_back({"scan", n, "hipref-vec"});
  }
  for (const char *n : {"n=1048576", "n=4194304"}) {
    rows.push_back({"fused_gelu", n, "hipref-naive"});
    rows.push_back({"fused_gelu", n, "hipref-vec"});
  }
  rows.push_back({"gemm", "m=512,n=512,k=512", "hipref-naive"});
  rows.push_back({"gemm", "m=1024,n=1024,k=1024", "hipref-naive"});
  return rows;
}

std::vector<Row> suite_rows(const std::string &suite) {
  std::vector<Row> rows;
  auto add = [&rows](const std::vector<Row> &more) { rows.insert(rows.end(), more.begin(), more.end()); };
  if (suite == "roofline" || suite == "all") {
    add({{"roofline_triad", "n=268435456", "roofline"}, {"roofline_fma", "n=4194304", "roofline"}});
  }
  if (suite == "kernelh" || suite == "all") add(kernelh_rows());
  if (suite == "rocblas" || suite == "all") add(gemm_rows("rocblas"));
  if (suite == "hipblaslt" || suite == "all") add(gemm_rows("hipblaslt"));
  if (suite == "hipref" || suite == "all") add(hipref_rows());
  return rows;
}

bool known_suite(const std::string &s) {
  return s == "all" || s == "roofline" || s == "kernelh" || s == "rocblas" || s == "hipblaslt" || s == "hipref";
}

// ---------------------------------------------------------------- occupancy

// One occupancy report (the reference's OccupancyReport, occupancy.cpp:90-110
// for its JSON keys): the analytic bound from the symbol the launcher runs at
// `shape` (its VGPR+AGPR count and static LDS) on the gfx950 limits entry,
// and, when a device is present, the vendor occupancy API on that loaded
// function. `threads` 0 takes the launcher's workgroup size at that shape.
struct OccupancyRow {
  std::string kernel, config, symbol;
  int32_t registers = 0, threads = 0;
  int64_t lds = 0;
  khrt_occupancy_report rep{};
};

const char *limiter_name(int32_t l) {
  static const char *names[] = {"none", "vgpr", "lds", "threads"};
  return l >= 0 && l <= 3 ? names[l] : "none";
}

// The reference's default shapes for the occupancy-only mode, used when no
// --shape is given (kernelh_backend.cpp:447-469); scan_totals as scan.
std::string default_occupancy_shape(const std::string &kernel) {
  static const std::map<std::string, std::string> shapes = {
      {"gemm", "m=512,n=512,k=512"},       {"softmax", "rows=4096,cols=1024"},
      {"layernorm", "rows=4096,cols=1024"}, {"scan", "n=100000"},
      {"scan_totals", "n=100000"},          {"fused_gelu", "n=1048576"},
      {"attention", "batch=2,heads=8,seq=512,head_dim=64"},
      {"vecadd", "n=1024"}};
  const auto it = shapes.find(kernel);
  return it == shapes.end() ? std::string() : it->second;
}

bool occupancy_row(const std::string &kernel, const std::string &shape, int threads, bool have_device,
                   OccupancyRow &row, std::string &error) {
  row.kernel = kernel;
  row.config = shape;
  char sym[64] = {0};
  khrt_kernel_resources r{};
  khrt_dim3 grid{}, block{};
  if (khrt_template_launch_symbol(kernel.c_str(), shape.c_str(), sym, sizeof(sym)) != 0 ||
      khrt_template_resources(sym, &r) != 0 ||
      khrt_template_geometry(kernel.c_str(), shape.c_str(), &grid, &block) != 0) {
    error = khrt_last_error();
    return false;
  }
  row.symbol = sym;
  row.registers = r.vgpr_count + r.agpr_count;
  row.lds = r.lds_bytes;
  row.threads = threads > 0 ? threads : static_cast<int32_t>(block.x * block.y * block.z);
  khrt_device_limits lim{};
  khrt_device_limits_for("gfx950", &lim);
  void *fn = nullptr;
  if (have_device && khrt_live_limits(&lim) != 0) return (error = khrt_last_error()), false;
  if (have_device) khrt_template_function(sym, &fn);
  const khrt_occupancy_input in{kernel.c_str(), "gfx950", shape.c_str(), row.registers, row.lds, row.threads};
  if (khrt_compute_occupancy(&in, &lim, fn, &row.rep) != 0) {
    error = khrt_last_error();
    return false;
  }
  return true;
}

std::string occupancy_json(const OccupancyRow &o, const std::string &indent) {
  std::ostringstream os;
  const std::string i2 = indent + "  ";
  os << "{\n"
     << i2 << "\"kernel\": \"" << json_escape(o.kernel) << "\",\n"
     << i2 << "\"target\": \"amdgcn-gfx950\",\n"
     << i2 << "\"config\": \"" << json_escape(o.config) << "\",\n"
     << i2 << "\"symbol\": \"" << json_escape(o.symbol) << "\",\n"
     << i2 << "\"vgpr_count\": " << o.registers << ",\n"
     << i2 << "\"lds_bytes\": " << o.lds << ",\n"
     << i2 << "\"threads_per_workgroup\": " << o.threads << ",\n"
     << i2 << "\"vgpr_limited_waves\": " << o.rep.vgpr_limited_waves << ",\n"
     << i2 << "\"lds_limited_blocks\": " << o.rep.lds_limited_blocks << ",\n"
     << i2 << "\"thread_limited_blocks\": " << o.rep.thread_limited_blocks << ",\n"
     << i2 << "\"theoretical_waves\": " << o.rep.achieved_waves << ",\n"
     << i2 << "\"theoretical_pct\": " << o.rep.theoretical_pct << ",\n"
     << i2 << "\"limiter\": \"" << limiter_name(o.rep.limiter) << "\",\n"
     << i2 << "\"measured_blocks\": " << o.rep.measured_blocks << ",\n"
     << i2 << "\"measured_pct\": " << o.rep.measured_pct << ",\n"
     << i2 << "\"measured_note\": \"" << json_escape(o.rep.measured_note) << "\"\n"
     << indent << "}";
  return os.str();
}

// occupancy.json (one report object, or {"reports": [...]} for a suite, as
// the reference writes them) and occupancy.md in `dir`.
bool write_occupancy(const fs::path &dir, const std::vector<OccupancyRow> &rows, bool single, std::string &error) {
  std::error_code ec;
  fs::create_directories(dir, ec);
  std::ofstream js(dir / "occupancy.json"), md(dir / "occupancy.md");
  if (!js || !md) {
    error = "cannot write occupancy files in '" + dir.string() + "'";
    return false;
  }
  if (single) {
    js << occupancy_json(rows.front(), "") << "\n";
  } else {
    js << "{\n  \"reports\": [\n";
    for (size_t i = 0; i < rows.size(); ++i)
      js << "    " << occupancy_json(rows[i], "    ") << (i + 1 < rows.size() ? ",\n" : "\n");
    js << "  ]\n}\n";
  }
  md << "# Occupancy report (gfx950)\n\n"
     << "Theoretical occupancy from the symbol the launcher runs at each shape (VGPR+AGPR count and\n"
     << "static LDS from its code-object notes) on the gfx950 device-limits entry; measured occupancy\n"
     << "from hipModuleOccupancyMaxActiveBlocksPerMultiprocessor on the loaded function when a device\n"
     << "is present.\n\n"
     << "| kernel | config | symbol | vgpr+agpr | lds (B) | threads | theoretical % | measured % | limiter |\n"
     << "| --- | --- | --- | ---: | ---: | ---: | ---: | ---: | --- |\n";
  for (const OccupancyRow &o : rows) {
    md << "| " << o.kernel << " | " << o.config << " | " << o.symbol << " | " << o.registers << " | " << o.lds
       << " | " << o.threads << " | " << o.rep.theoretical_pct << " | ";
    if (o.rep.measured_blocks >= 0) {
      md << o.rep.measured_pct;
    } else {
      md << "n/a";
    }
    md << " | " << limiter_name(o.rep.limiter) << " |\n";
  }
  md << "\nNotes:\n"
     << "- achieved_waves = min(VGPR-limited waves, LDS-limited blocks, thread-limited blocks), the three\n"
     << "  bounds compared directly as the reference's formula pins them; theoretical % = achieved_waves /\n"
     << "  waves_per_cu x 100 (waves_per_cu = 32 on gfx950).\n"
     << "- measured % = resident blocks x waves per block / waves_per_cu x 100 from the vendor API; n/a\n"
     << "  without a device.\n";
  std::cout << "wrote " << (dir / "occupancy.json").string() << "\nwrote " << (dir / "occupancy.md").string()
            << "\n";
  return true;
}

// Occupancy of every kernelh row of the given rows (the reference writes
// one report per kernelh row of the suite, kernelh_backend.cpp:658-698).
int write_suite_occupancy(const fs::path &dir, const std::vector<Row> &rows, bool have_device) {
  std::vector<OccupancyRow> out;
  for (const Row &row : rows) {
    if (row.backend != "kernelh") continue;
    OccupancyRow o;
    std::string error;
    if (!occupancy_row(row.kernel, row.shape, 0, have_device, o, error)) {
      std::cerr << "error: occupancy " << row.kernel << " " << row.shape << ": " << error << "\n";
      return kExitOperational;
    }
    out.push_back(o);
  }
  if (out.empty()) {
    std::cerr << "error: no kernelh rows for occupancy\n";
    return kExitOperational;
  }
  std::string error;
  if (!write_occupancy(dir, out, false, error)) {
    std::cerr << "error: " << error << "\n";
    return kExitOperational;
  }
  return kExitOk;
}

bool device_present() {
  int n = 0;
  return khrt_device_count(&n) == 0 && n > 0 && khrt_init_device(0) == 0;
}

// `bench --occupancy --kernel <k> --target amdgcn-gfx950 [--shape ...]
// [--threads N] --out <dir>`: occupancy.{json,md} for one kernel and shape,
// timing nothing; no device needed (run_bench.cpp:111-127).
int run_occupancy_only(const std::string &kernel, const std::string &shape_in, int threads, const fs::path &dir) {
  const std::string shape = shape_in.empty() ? default_occupancy_shape(kernel) : shape_in;
  if (shape.empty()) {
    std::cerr << "error: unknown kernel '" << kernel << "' for --occupancy (no default shape); use --shape k=v,...\n";
    return kExitOperational;
  }
  OccupancyRow o;
  std::string error;
  if (!occupancy_row(kernel, shape, threads, device_present(), o, error) || !write_occupancy(dir, {o}, true, error)) {
    std::cerr << "error: " << error << "\n";
    return kExitOperational;
  }
  std::cout << "wrote " << dir.string() << "/occupancy.json + occupancy.md (" << kernel << ", amdgcn-gfx950)\n";
  return kExitOk;
}

int run_bench(int argc, char **argv) {
  std::string suite = "all", out, kernel, shape, backend = "kernelh", target;
  long warmup = 5, iters = 20, threads = 0;
  bool occupancy = false, ok = true;
  for (khcli::ArgCursor a(argc, argv, 2); !a.done() && ok;) {
    if (a.flag("--help") || a.flag("-h")) {
      usage(std::cout);
      return kExitOk;
    }
    if (a.value("--suite", suite) || a.value("--out", out) || a.value("--kernel", kernel) ||
        a.value("--shape", shape) || a.value("--backend", backend) || a.value("--target", target) ||
        a.integer("--warmup", 0, 1000000, warmup, ok) || a.integer("--iters", 1, 1000000, iters, ok) ||
        a.integer("--threads", 1, 1048576, threads, ok)) {
      continue;
    }
    if (a.flag("--occupancy")) {
      occupancy = true;
      continue;
    }
    std::cerr << "error: unknown bench option '" << a.word() << "'\n";
    return kExitUsage;
  }
  if (!ok) return kExitUsage;
  if (out.empty()) {
    std::cerr << "error: bench requires --out <path> (a .csv file or a dir)\n";
    return kExitUsage;
  }
  kernelh::ShapeDims dims;
  std::string why;
  if (!shape.empty() && !kernelh::parse_shape_text(shape, dims, &why)) {
    std::cerr << "error: malformed --shape: expected " << why << "\n";
    return kExitUsage;
  }
  // The reference's occupancy-only mode (--occupancy --kernel --target);
  // --target and --threads belong to it alone.
  if ((!target.empty() || threads != 0) && !(occupancy && !kernel.empty())) {
    std::cerr << "error: --target/--threads require --occupancy --kernel <name>\n";
    return kExitUsage;
  }
  if (occupancy && !kernel.empty() && !target.empty()) {
    if (target != "amdgcn-gfx950") {
      std::cerr << "error: unknown --target '" << target << "' for --occupancy\n"
                << "error: valid --target values: amdgcn-gfx950\n";
      return kExitUsage;
    }
    return run_occupancy_only(kernel, shape, static_cast<int>(threads), fs::path(out));
  }
  // Otherwise --kernel times one row at --shape (with its occupancy when
  // --occupancy is given); --occupancy --kernel alone names no shape.
  if (!kernel.empty() && shape.empty()) {
    std::cerr << "error: --kernel needs --shape to time a row, or --occupancy --kernel <name> --target "
                 "amdgcn-gfx950 for its occupancy alone\n";
    return kExitUsage;
  }
  const bool known_backend = backend == "kernelh" || backend == "rocblas" || backend == "hipblaslt" ||
                             backend == "hipref-naive" || backend == "hipref-vec" || backend == "roofline";
  if (!known_suite(suite) || !known_backend) {
    std::cerr << "error: bench takes a suite of roofline|kernelh|rocblas|hipblaslt|hipref|all and a backend of "
                 "kernelh|rocblas|hipblaslt|hipref-naive|hipref-vec|roofline\n";
    return kExitUsage;
  }
  fs::path csv = out;
  std::error_code ec;
  if (csv.extension() != ".csv") {
    fs::create_directories(csv, ec);
    csv /= "results.csv";
  } else if (csv.has_parent_path()) {
    fs::create_directories(csv.parent_path(), ec);
  }
  const fs::path dir = csv.has_parent_path() ? csv.parent_path() : fs::path(".");
  std::vector<Row> rows = kernel.empty() ? suite_rows(suite) : std::vector<Row>{{kernel, shape, backend}};
  if (!device_present()) {
    std::cerr << "skip: no HIP device available (" << khrt_last_error() << ")\n";
    if (occupancy) write_suite_occupancy(dir, rows, false);
    return kExitSkip;
  }
  khrt_device_info info{};
  khrt_get_device_info(&info);
  const std::string device = std::string(info.name[0] ? info.name : "AMD Instinct MI355X") + " (" + info.arch + ")";
  const bool fresh = !fs::exists(csv);
  std::ofstream f(csv, std::ios::app);
  if (fresh) f << "kernel,shape,backend,ms_median,gflops_or_gbps,timestamp,device\n";
  int failures = 0;
  for (const Row &row : rows) {
    Bufs b;
    std::function<int()> launch;
    double work = 0.0;
    bool flops = false;
    double ms = 0.0;
    std::string error;
    if (!prepare(row, b, launch, work, flops, error)) {
      std::cerr << "error: " << row.backend << " " << row.kernel << " " << row.shape << ": " << error << "\n";
      ++failures;
      continue;
    }
    if (!time_row(launch, static_cast<int>(warmup), static_cast<int>(iters), ms)) {
      std::cerr << "error: " << row.backend << " " << row.kernel << " " << row.shape << ": " << khrt_last_error()
                << "\n";
      ++failures;
      continue;
    }
    double rate = 0.0;
    const double args[2] = {work, ms};
    khrt_bench_metric(flops ? "gflops_from_ms" : "gbps_from_ms", args, 2, &rate);
    std::string shp = row.shape;
    std::replace(shp.begin(), shp.end(), ',', ';');
    f << row.kernel << "," << shp << "," << row.backend << "," << ms << "," << rate << "," << now_iso() << ",\""
      << device << "\"\n";
    std::printf("%-13s %-15s %-40s %10.4f ms %12.1f %s\n", row.backend.c_str(), row.kernel.c_str(),
                row.shape.c_str(), ms, rate, flops ? "GFLOP/s" : "GB/s");
  }
  std::cout << "wrote " << csv.string() << "\n";
  if (occupancy && write_suite_occupancy(dir, rows, true) != kExitOk) ++failures;
  return failures ? kExitOperational : kExitOk;
}

int run_info() {
  khrt_device_limits l{};
  khrt_device_limits_for("gfx950", &l);
  std::printf("table gfx950: %s lds=%lld wave=%d max_threads=%d waves_per_cu=%d reg_file=%d\n", l.name,
              (long long)l.lds_bytes_per_workgroup, l.wavefront_size, l.max_threads_per_workgroup, l.waves_per_cu,
              l.reg_file_per_cu);
  int n = 0;
  if (khrt_device_count(&n) != 0 || n < 1) {
    std::printf("no HIP device\n");
    return kExitSkip;
  }
  khrt_device_info d{};
  if (khrt_get_device_info(&d) != 0) {
    std::fprintf(stderr, "error: %s\n", khrt_last_error());
    return kExitOperational;
  }
  std::printf("device 0: %s arch=%s cu=%lld lds=%lld wave=%d vram=%lld B\n", d.name, d.arch, (long long)d.cu_count,
              (long long)d.lds_bytes_per_workgroup, d.wavefront_size, (long long)d.vram_bytes);
  return kExitOk;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc < 2) {
    usage(std::cerr);
    return kExitUsage;
  }
  const std::string cmd = argv[1];
  if (cmd == "--help" || cmd == "-h") {
    usage(std::cout);
    return kExitOk;
  }
  if (cmd == "compile") {
    if (argc == 2) {
      usage(std::cerr);
      return kExitUsage;
    }
    return run_compile(argc, argv);
  }
  if (cmd == "bench") return run_bench(argc, argv);
  if (cmd == "tune") return khcli::run_tune(argc, argv);
  if (cmd == "tune-eval") return khcli::run_tune_eval(argc, argv);
  if (cmd == "info") return run_info();
  std::cerr << "error: unknown command '" << cmd << "'\n";
  usage(std::cerr);
  return kExitUsage;
}
