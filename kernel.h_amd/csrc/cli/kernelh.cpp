// kernelh - command-line driver for the gfx950 kernel.h templates.
//
// The reference's CLI surface for this path (tools/kernelh/main.cpp):
//   kernelh compile --kernel <name> --shape k=v,... --target <t> --out <dir>
//                   [--resources]                          (main.cpp:435-646)
//   kernelh tune    --kernel gemm --shape m=..,n=..,k=.. --out <dir> [...]
//                                                          (main.cpp:649-1420)
//   kernelh bench   --suite <roofline|kernelh|rocblas|hipblaslt|hipref|all> --out <path>
//                   [--occupancy] [--kernel <name> --shape ... [--backend <b>]]
//                                                          (main.cpp:2154-2228)
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

#include "comparators.hpp"
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
     << "  --shape m=..,n=..,k=.. --out <dir> [--max-candidates n] [--timeout s]\n"
     << "  [--cache path]; writes <dir>/tune-results.csv, prints the best config\n\n"
     << "bench options:\n"
     << "  --suite <name>        roofline, kernelh, rocblas, hipblaslt, hipref, all (default: all)\n"
     << "  --backend <name>      with --kernel: kernelh (default), rocblas, hipblaslt,\n"
     << "                        hipref-naive, hipref-vec, roofline\n"
     << "  --kernel <name>       single-row mode: time one template ...\n"
     << "  --shape k=v,...       ... at this shape\n"
     << "  --out <path>          results.csv path or directory (required)\n"
     << "  --warmup <n>          warmup launches (default 5)\n"
     << "  --iters <n>           timed launches, median reported (default 20)\n"
     << "  --occupancy           write occupancy.{json,md} next to results.csv\n\n"
     << "info                    print the live device and the gfx950 limits entry\n\n"
     << "--help prints this usage and exits 0.\n";
}

bool take(int argc, char **argv, int &i, const std::string &arg, const char *flag, std::string &out) {
  const std::string prefix = std::string(flag) + "=";
  if (arg.rfind(prefix, 0) == 0) {
    out = arg.substr(prefix.size());
    return true;
  }
  if (arg == flag) {
    if (i + 1 >= argc) {
      std::cerr << "error: " << flag << " requires a value\n";
      std::exit(kExitUsage);
    }
    out = argv[++i];
    return true;
  }
  return false;
}

bool parse_shape(const std::string &text, std::map<std::string, int64_t> &shape) {
  size_t start = 0;
  while (start <= text.size()) {
    const size_t comma = text.find(',', start);
    const size_t end = comma == std::string::npos ? text.size() : comma;
    const std::string item = text.substr(start, end - start);
    const size_t eq = item.find('=');
    if (eq == std::string::npos || eq == 0 || eq + 1 >= item.size()) return false;
    char *vend = nullptr;
    errno = 0;
    const long long v = std::strtoll(item.c_str() + eq + 1, &vend, 10);
    if (errno != 0 || *vend != '\0') return false;
    shape[item.substr(0, eq)] = v;
    if (comma == std::string::npos) break;
    start = comma + 1;
  }
  return true;
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
  bool resources = false, have_target = false;
  for (int i = 2; i < argc; ++i) {
    const std::string arg = argv[i];
    std::string v;
    if (arg == "--help" || arg == "-h") {
      usage(std::cout);
      return kExitOk;
    } else if (take(argc, argv, i, arg, "--kernel", v)) {
      kernel = v;
    } else if (take(argc, argv, i, arg, "--shape", v)) {
      shape = v;
    } else if (take(argc, argv, i, arg, "--target", v)) {
      target = v;
      have_target = true;
    } else if (take(argc, argv, i, arg, "--out", v)) {
      out = v;
    } else if (arg == "--resources") {
      resources = true;
    } else {
      std::cerr << "error: unknown compile option '" << arg << "'\n";
      usage(std::cerr);
      return kExitUsage;
    }
  }
  (void)have_target;
  if (kernel.empty() || shape.empty() || out.empty()) {
    std::cerr << "error: compile needs --kernel, --shape and --out\n";
    usage(std::cerr);
    return kExitUsage;
  }
  std::map<std::string, int64_t> parsed;
  if (!parse_shape(shape, parsed)) {
    std::cerr << "error: malformed --shape '" << shape << "'\n";
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

// Allocates the row's buffers and returns a launcher closure. Rates use the
// reference's formulas (bench/harness/metrics.cpp), so rows compare across
// backends: bytes for the bandwidth kernels, 2mnk / 4bhs^2d FLOPs.
bool prepare(const Row &row, Bufs &b, std::function<int()> &launch, double &work, bool &flops, std::string &error) {
  std::map<std::string, int64_t> s;
  if (!parse_shape(row.shape, s)) {
    error = "malformed shape";
    return false;
  }
  const std::string &k = row.kernel;
  flops = false;
  if (row.backend == "hipref-naive" || row.backend == "hipref-vec") {
    return khcli::prepare_hipref(k, row.backend == "hipref-vec" ? "vec4" : "naive", s, b, launch, work, flops, error);
  }
  if (row.backend == "rocblas") {
    if (k != "gemm") {
      error = "rocblas backend only benchmarks gemm (got '" + k + "')";
      return false;
    }
    flops = true;
    return khcli::prepare_rocblas_gemm(s, b, launch, work, error);
  }
  if (row.backend == "hipblaslt") {
    if (k != "gemm") {
      error = "hipblaslt backend only benchmarks gemm (got '" + k + "')";
      return false;
    }
    flops = true;
    return khcli::prepare_hipblaslt_gemm(s, b, launch, work, error);
  }
  if (k == "roofline_fma") {
    flops = true;
    return khcli::prepare_roofline_fma(b, launch, work, error);
  }
  error = "unknown kernel or allocation failure";
  if (k == "vecadd") {
    const int64_t n = get(s, "n");
    float *a = b.alloc(n, 1.0f), *bb = b.alloc(n, 2.0f), *c = b.alloc(n, 0.0f);
    launch = [=] { return kh_vecadd(a, bb, c, n, nullptr); };
    work = 12.0 * n;
  } else if (k == "fused_gelu") {
    const int64_t n = s.count("n") ? get(s, "n") : get(s, "rows") * get(s, "cols");
    float *x = b.alloc(n, 0.25f), *o = b.alloc(n, 0.0f);
    launch = [=] { return kh_fused_gelu(x, nullptr, o, n, nullptr); };
    work = 12.0 * n;  // fused_gelu_bytes counts the (dead) tmp stream too
  } else if (k == "softmax" || k == "layernorm") {
    const int64_t r = get(s, "rows"), c = get(s, "cols");
    float *x = b.alloc(r * c, 0.5f), *y = b.alloc(r * c, 0.0f);
    if (k == "softmax") {
      launch = [=] { return kh_softmax(x, y, r, c, nullptr); };
      work = 8.0 * r * c;
    } else {
      float *g = b.alloc(c, 1.0f), *bt = b.alloc(c, 0.0f);
      launch = [=] { return kh_layernorm(x, g, bt, y, r, c, nullptr); };
      work = 8.0 * r * c + 8.0 * c;
    }
  } else if (k == "scan") {
    const int64_t n = get(s, "n"), T = (n + 255) / 256;
    float *x = b.alloc(n, 0.5f), *y = b.alloc(n, 0.0f), *th = b.alloc(T, 0.0f), *tl = b.alloc(T, 0.0f);
    launch = [=] { return kh_scan(x, y, nullptr, th, tl, n, nullptr); };
    work = 8.0 * n;
  } else if (k == "gemm") {
    const int64_t m = get(s, "m"), n = get(s, "n"), kk = get(s, "k");
    float *A = b.alloc(m * kk, 1.0f), *B = b.alloc(kk * n, 1.0f), *C = b.alloc(m * n, 0.0f);
    launch = [=] { return kh_gemm(A, B, C, m, n, kk, nullptr); };
    work = 2.0 * m * n * kk;
    flops = true;
  } else if (k == "attention") {
    const int64_t bt = get(s, "batch"), h = get(s, "heads"), sq = get(s, "seq"), d = get(s, "head_dim", 64);
    const int64_t e = bt * h * sq * d;
    float *Q = b.alloc(e, 0.01f), *K = b.alloc(e, 0.02f), *V = b.alloc(e, 1.0f), *O = b.alloc(e, 0.0f);
    launch = [=] { return kh_attention(Q, K, V, O, bt, h, sq, d, nullptr); };
    work = 4.0 * bt * h * sq * sq * d;
    flops = true;
  } else if (k == "roofline_triad") {
    const int64_t n = get(s, "n");
    float *a = b.alloc(n, 1.0f), *bb = b.alloc(n, 2.0f), *c = b.alloc(n, 0.0f);
    launch = [=] { return kh_roofline_triad(a, bb, c, n, nullptr); };
    work = 12.0 * n;
  } else {
    return false;
  }
  for (void *p : b.ptrs)
    if (p == nullptr) return false;
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

int write_occupancy(const fs::path &dir, const std::vector<std::string> &kernels) {
  std::ofstream js(dir / "occupancy.json"), md(dir / "occupancy.md");
  md << "# Occupancy report (gfx950)\n\n"
     << "achieved_waves = min(VGPR-limited waves, LDS-limited blocks, thread-limited blocks) on the\n"
     << "gfx950 device-limits entry; measured % from the vendor occupancy API when a device is\n"
     << "present.\n\n| kernel | vgpr+agpr | lds (B) | block | theoretical % | measured % | limiter |\n"
     << "| --- | ---: | ---: | ---: | ---: | ---: | --- |\n";
  js << "{\n  \"reports\": [\n";
  const char *limiters[] = {"none", "vgpr", "lds", "threads"};
  khrt_device_limits lim{};
  khrt_device_limits_for("gfx950", &lim);
  int dev_count = 0;
  const bool have_dev = khrt_device_count(&dev_count) == 0 && dev_count > 0;
  if (have_dev) khrt_live_limits(&lim);
  for (size_t i = 0; i < kernels.size(); ++i) {
    const std::string &k = kernels[i];
    khrt_kernel_resources r{};
    if (khrt_template_resources(k.c_str(), &r) != 0) continue;
    const int block = (k == "scan") ? 1024 : 256;
    void *fn = nullptr;
    if (have_dev) khrt_template_function(k.c_str(), &fn);
    khrt_occupancy_input in{k.c_str(), "gfx950", "", r.vgpr_count + r.agpr_count, r.lds_bytes, block};
    khrt_occupancy_report rep{};
    khrt_compute_occupancy(&in, &lim, fn, &rep);
    js << "    {\"kernel\": \"" << k << "\", \"vgpr_count\": " << r.vgpr_count + r.agpr_count
       << ", \"lds_bytes\": " << r.lds_bytes << ", \"threads_per_workgroup\": " << block
       << ", \"theoretical_waves\": " << rep.achieved_waves << ", \"theoretical_pct\": " << rep.theoretical_pct
       << ", \"limiter\": \"" << limiters[rep.limiter] << "\", \"measured_blocks\": " << rep.measured_blocks
       << ", \"measured_pct\": " << rep.measured_pct << "}" << (i + 1 < kernels.size() ? "," : "") << "\n";
    md << "| " << k << " | " << r.vgpr_count + r.agpr_count << " | " << r.lds_bytes << " | " << block << " | "
       << rep.theoretical_pct << " | ";
    if (rep.measured_blocks >= 0) {
      md << rep.measured_pct;
    } else {
      md << "n/a";
    }
    md << " | " << limiters[rep.limiter] << " |\n";
  }
  js << "  ]\n}\n";
  std::cout << "wrote " << (dir / "occupancy.json").string() << "\nwrote " << (dir / "occupancy.md").string() << "\n";
  return kExitOk;
}

int run_bench(int argc, char **argv) {
  std::string suite = "all", out, kernel, shape, backend = "kernelh", v;
  int warmup = 5, iters = 20;
  bool occupancy = false;
  for (int i = 2; i < argc; ++i) {
    const std::string arg = argv[i];
    if (arg == "--help" || arg == "-h") {
      usage(std::cout);
      return kExitOk;
    } else if (take(argc, argv, i, arg, "--suite", v)) {
      suite = v;
    } else if (take(argc, argv, i, arg, "--out", v)) {
      out = v;
    } else if (take(argc, argv, i, arg, "--kernel", v)) {
      kernel = v;
    } else if (take(argc, argv, i, arg, "--shape", v)) {
      shape = v;
    } else if (take(argc, argv, i, arg, "--backend", v)) {
      backend = v;
    } else if (take(argc, argv, i, arg, "--warmup", v)) {
      warmup = std::atoi(v.c_str());
    } else if (take(argc, argv, i, arg, "--iters", v)) {
      iters = std::atoi(v.c_str());
    } else if (arg == "--occupancy") {
      occupancy = true;
    } else {
      std::cerr << "error: unknown bench option '" << arg << "'\n";
      return kExitUsage;
    }
  }
  const bool known_backend = backend == "kernelh" || backend == "rocblas" || backend == "hipblaslt" ||
                             backend == "hipref-naive" || backend == "hipref-vec" || backend == "roofline";
  if (out.empty() || !known_suite(suite) || !known_backend || iters < 1 || warmup < 0 ||
      (!kernel.empty() && shape.empty())) {
    std::cerr << "error: bench needs --out, a suite of roofline|kernelh|rocblas|hipblaslt|hipref|all, a backend of "
                 "kernelh|rocblas|hipblaslt|hipref-naive|hipref-vec|roofline, and --shape with --kernel\n";
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
  int n = 0;
  if (khrt_device_count(&n) != 0 || n < 1 || khrt_init_device(0) != 0) {
    std::cerr << "skip: no HIP device available (" << khrt_last_error() << ")\n";
    if (occupancy) write_occupancy(csv.parent_path(), {"vecadd", "gemm", "softmax", "layernorm", "scan", "scan_totals",
                                                       "fused_gelu", "attention"});
    return kExitSkip;
  }
  khrt_device_info info{};
  khrt_get_device_info(&info);
  const std::string device = std::string(info.name[0] ? info.name : "AMD Instinct MI355X") + " (" + info.arch + ")";
  std::vector<Row> rows = kernel.empty() ? suite_rows(suite) : std::vector<Row>{{kernel, shape, backend}};
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
    if (!time_row(launch, warmup, iters, ms)) {
      std::cerr << "error: " << row.backend << " " << row.kernel << " " << row.shape << ": " << khrt_last_error()
                << "\n";
      ++failures;
      continue;
    }
    const double rate = work * 1000.0 / ms / 1e9;  // GFLOP/s or GB/s (metrics.cpp:5-12)
    std::string shp = row.shape;
    std::replace(shp.begin(), shp.end(), ',', ';');
    f << row.kernel << "," << shp << "," << row.backend << "," << ms << "," << rate << "," << now_iso() << ",\""
      << device << "\"\n";
    std::printf("%-13s %-15s %-40s %10.4f ms %12.1f %s\n", row.backend.c_str(), row.kernel.c_str(),
                row.shape.c_str(), ms, rate, flops ? "GFLOP/s" : "GB/s");
  }
  std::cout << "wrote " << csv.string() << "\n";
  if (occupancy) {
    write_occupancy(csv.parent_path(),
                    kernel.empty() ? std::vector<std::string>{"vecadd", "gemm", "softmax", "layernorm", "scan",
                                                              "scan_totals", "fused_gelu", "attention"}
                                   : std::vector<std::string>{kernel});
  }
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
