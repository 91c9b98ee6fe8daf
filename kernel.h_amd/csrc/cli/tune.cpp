// `kernelh tune`: GEMM tile autotune over the gfx950 candidate space
// (gemm_tune_list.h), with the reference's evaluator contract
// (tools/kernelh/main.cpp:649-673, 1320-1420; lib/compiler/autotuner.cpp):
//   * every candidate is evaluated in a child process with a wall-clock
//     deadline; a hung or crashed candidate is recorded ("timeout",
//     "crashed") and never hangs the run. The parent never initialises HIP:
//     it starts `kernelh tune-eval` children, each of which does;
//   * the child re-verifies the candidate on a small shape (each dimension
//     capped at 128) against an fp64 host product, relative Frobenius
//     <= 1e-5, then times it at the tuning shape: warmup 3, median of 10;
//   * results go to <out>/tune-results.csv (the reference's columns, then
//     symbol, wave_tile, prio, lds_dma, gflops) and to a cache file keyed by
//     kernel|shape|device, so a second run with the same key is served from
//     the cache.
// Differences, each stated in the usage text: the space is a fixed set of
// precompiled instantiations (no per-candidate compilation), so it is
// evaluated exhaustively up to --max-candidates instead of sampled and
// refined, and the cache key is an FNV-1a 64-bit hash.
#include "tune.hpp"

#include "khrt.h"
#include "gemm_tune_list.h"

#include <poll.h>
#include <signal.h>
#include <spawn.h>
#include <sys/wait.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

extern char **environ;

// The candidate code object, embedded by build.py (gen/kh_cli_embed.S).
extern "C" const unsigned char kh_cli_co_gemm_tune[];
extern "C" const unsigned char kh_cli_co_gemm_tune_end[];

namespace khcli {
namespace {

namespace fs = std::filesystem;

struct Candidate {
  int wtm, wtn, bk, prio, dma;
  const char *symbol;
  int bm() const { return 64 * wtm; }
  int bn() const { return 64 * wtn; }
};

#define KH_STR2(x) #x
#define KH_STR(x) KH_STR2(x)
#define KH_TUNE_ROW(WTM, WTN, BK, PRIO, DMA) \
  {WTM, WTN, BK, PRIO, DMA, KH_STR(KH_GEMM_TUNE_SYMBOL(WTM, WTN, BK, PRIO, DMA))},
const Candidate kCandidates[] = {KH_GEMM_TUNE_CONFIGS(KH_TUNE_ROW)};
#undef KH_TUNE_ROW

struct Result {
  const Candidate *c = nullptr;
  bool accepted = false;
  double ms = 0.0;
  double gflops = 0.0;
  std::string reason;
};

bool take(int argc, char **argv, int &i, const std::string &arg, const char *flag, std::string &out) {
  if (arg == flag && i + 1 < argc) {
    out = argv[++i];
    return true;
  }
  const std::string pre = std::string(flag) + "=";
  if (arg.rfind(pre, 0) == 0) {
    out = arg.substr(pre.size());
    return true;
  }
  return false;
}

bool parse_mnk(const std::string &text, int64_t &m, int64_t &n, int64_t &k) {
  m = n = k = 0;
  std::stringstream ss(text);
  std::string item;
  while (std::getline(ss, item, ',')) {
    const auto eq = item.find('=');
    if (eq == std::string::npos) return false;
    char *end = nullptr;
    const long long v = std::strtoll(item.c_str() + eq + 1, &end, 10);
    if (*end != '\0') return false;
    const std::string key = item.substr(0, eq);
    if (key == "m") m = v;
    else if (key == "n") n = v;
    else if (key == "k") k = v;
    else return false;
  }
  return m > 0 && n > 0 && k > 0;
}

std::string fnv1a_hex(const std::string &s) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ull;
  }
  char buf[17];
  std::snprintf(buf, sizeof buf, "%016llx", static_cast<unsigned long long>(h));
  return buf;
}

std::string self_exe() {
  char buf[4096];
  const ssize_t n = ::readlink("/proc/self/exe", buf, sizeof(buf) - 1);
  if (n <= 0) return "kernelh";
  buf[n] = '\0';
  return buf;
}

// Runs `args` as a child with stdout captured; kills it after `timeout_s`.
// Returns the captured output; `status` gets the wait status, `timed_out`
// whether the deadline fired.
std::string run_child(const std::vector<std::string> &args, int timeout_s, int &status, bool &timed_out) {
  status = 0;
  timed_out = false;
  int fds[2];
  if (::pipe(fds) != 0) return "";
  posix_spawn_file_actions_t fa;
  posix_spawn_file_actions_init(&fa);
  posix_spawn_file_actions_adddup2(&fa, fds[1], STDOUT_FILENO);
  posix_spawn_file_actions_addclose(&fa, fds[0]);
  std::vector<char *> argv;
  for (const std::string &a : args) argv.push_back(const_cast<char *>(a.c_str()));
  argv.push_back(nullptr);
  pid_t pid = 0;
  const int rc = posix_spawn(&pid, argv[0], &fa, nullptr, argv.data(), environ);
  posix_spawn_file_actions_destroy(&fa);
  ::close(fds[1]);
  if (rc != 0) {
    ::close(fds[0]);
    status = -1;
    return "";
  }
  std::string out;
  const auto deadline = std::chrono::steady_clock::now() + std::chrono::seconds(timeout_s);
  char buf[4096];
  for (;;) {
    const auto left = std::chrono::duration_cast<std::chrono::milliseconds>(deadline - std::chrono::steady_clock::now());
    if (left.count() <= 0) {
      timed_out = true;
      ::kill(pid, SIGKILL);
      break;
    }
    pollfd p{fds[0], POLLIN, 0};
    const int pr = ::poll(&p, 1, static_cast<int>(std::min<long long>(left.count(), 1000)));
    if (pr < 0 && errno != EINTR) break;
    if (pr > 0) {
      const ssize_t n = ::read(fds[0], buf, sizeof buf);
      if (n <= 0) break;  // child closed stdout (exited)
      out.append(buf, static_cast<size_t>(n));
    }
  }
  ::close(fds[0]);
  ::waitpid(pid, &status, 0);
  return out;
}

// Value of `key=` on the RESULT line a child printed ("" when absent).
std::string field(const std::string &out, const std::string &key) {
  const auto line = out.rfind("RESULT ");
  if (line == std::string::npos) return "";
  const auto eol = out.find('\n', line);
  const std::string l = out.substr(line, eol == std::string::npos ? std::string::npos : eol - line);
  const auto at = l.find(" " + key + "=");
  if (at == std::string::npos) return "";
  const auto start = at + key.size() + 2;
  if (key == "reason") return l.substr(start);  // reason runs to the end of the line
  const auto end = l.find(' ', start);
  return l.substr(start, end == std::string::npos ? std::string::npos : end - start);
}

std::string csv_escape(const std::string &s) {
  if (s.find_first_of(",\"\n") == std::string::npos) return s;
  std::string o = "\"";
  for (char c : s) {
    if (c == '"') o += '"';
    o += c;
  }
  return o + "\"";
}

std::string json_escape(const std::string &s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') {
      o += '\\';
      o += c;
    } else if (c == '\n') {
      o += "\\n";
    } else {
      o += c;
    }
  }
  return o;
}

std::string json_unescape(const std::string &s) {
  std::string o;
  for (size_t i = 0; i < s.size(); ++i) {
    if (s[i] == '\\' && i + 1 < s.size()) {
      ++i;
      o += s[i] == 'n' ? '\n' : s[i];
    } else {
      o += s[i];
    }
  }
  return o;
}

// The cache: one JSON object per line, {"key": ..., "best": ..., "csv": ...}.
bool cache_lookup(const std::string &path, const std::string &key, std::string &best, std::string &csv) {
  std::ifstream f(path);
  std::string line;
  const std::string tag = "{\"key\": \"" + key + "\"";
  while (std::getline(f, line)) {
    if (line.rfind(tag, 0) != 0) continue;
    const auto b = line.find("\"best\": \"");
    const auto c = line.find("\"csv\": \"");
    if (b == std::string::npos || c == std::string::npos) continue;
    best = line.substr(b + 9, line.find('"', b + 9) - (b + 9));
    csv = json_unescape(line.substr(c + 8, line.rfind('"') - (c + 8)));
    return true;
  }
  return false;
}

void cache_store(const std::string &path, const std::string &key, const std::string &best, const std::string &csv) {
  std::error_code ec;
  if (fs::path(path).has_parent_path()) fs::create_directories(fs::path(path).parent_path(), ec);
  std::ofstream f(path, std::ios::app);
  f << "{\"key\": \"" << key << "\", \"best\": \"" << best << "\", \"csv\": \"" << json_escape(csv) << "\"}\n";
}

void usage_tune(std::ostream &os) {
  os << "usage: kernelh tune --kernel gemm --shape m=..,n=..,k=.. --out <dir> [options]\n"
     << "  --target <t>          amdgcn-gfx950 (default; the local execution target)\n"
     << "  --max-candidates <n>  cap on evaluated candidates (1..80, default 80)\n"
     << "  --timeout <seconds>   wall clock per candidate (1..3600, default 30)\n"
     << "  --cache <path>        cache file (default build/tune-cache.json), keyed\n"
     << "                        FNV-1a(kernel|shape|device)\n"
     << "The space (KH_GEMM_TUNE_CONFIGS) is a fixed set of precompiled gfx950\n"
     << "instantiations: wave tile WTM x WTN of 32x32 MFMAs, slab depth BK, MFMA\n"
     << "wave priority and slab pipeline (register-staged, or direct-to-LDS with three\n"
     << "stages); it is evaluated exhaustively, not sampled.\n";
}

// ---------------------------------------------------------------- child

// Deterministic U[-1,1) fill (64-bit LCG, top 24 bits).
void fill_uniform(std::vector<float> &v, uint64_t seed) {
  for (float &x : v) {
    seed = seed * 6364136223846793005ull + 1442695040888963407ull;
    x = static_cast<float>(static_cast<double>(seed >> 40) / 8388608.0 - 1.0);
  }
}

void fill_args(void *A, void *B, void *C, int64_t m, int64_t n, int64_t k, std::vector<uint64_t> &slots,
               std::vector<void *> &params) {
  slots.assign(21, 0);
  size_t i = 0;
  auto memref2 = [&](void *p, int64_t r, int64_t c) {
    slots[i++] = reinterpret_cast<uint64_t>(p);
    slots[i++] = reinterpret_cast<uint64_t>(p);
    slots[i++] = 0;
    slots[i++] = static_cast<uint64_t>(r);
    slots[i++] = static_cast<uint64_t>(c);
    slots[i++] = static_cast<uint64_t>(c);
    slots[i++] = 1;
  };
  memref2(A, m, k);
  memref2(B, k, n);
  memref2(C, m, n);
  params.clear();
  for (uint64_t &s : slots) params.push_back(&s);
}

int eval_print(bool accepted, double ms, double gflops, const std::string &reason) {
  std::printf("RESULT accepted=%d ms=%.6f gflops=%.1f reason=%s\n", accepted ? 1 : 0, ms, gflops, reason.c_str());
  std::fflush(stdout);
  return 0;
}

}  // namespace

int run_tune_eval(int argc, char **argv) {
  std::string symbol, shape, v;
  int bm = 0, bn = 0;
  bool probe = false;
  for (int i = 2; i < argc; ++i) {
    const std::string arg = argv[i];
    if (take(argc, argv, i, arg, "--symbol", v)) symbol = v;
    else if (take(argc, argv, i, arg, "--shape", v)) shape = v;
    else if (take(argc, argv, i, arg, "--bm", v)) bm = std::atoi(v.c_str());
    else if (take(argc, argv, i, arg, "--bn", v)) bn = std::atoi(v.c_str());
    else if (arg == "--probe") probe = true;
  }
  int count = 0;
  if (khrt_device_count(&count) != 0 || count < 1 || khrt_init_device(0) != 0) {
    return eval_print(false, 0, 0, "skip: no HIP device");
  }
  if (probe) {
    khrt_device_info info{};
    khrt_get_device_info(&info);
    std::printf("DEVICE %s (%s) cu=%lld\n", info.name[0] ? info.name : "AMD Instinct MI355X", info.arch,
                static_cast<long long>(info.cu_count));
    return 0;
  }
  int64_t m, n, k;
  if (symbol.empty() || bm <= 0 || bn <= 0 || !parse_mnk(shape, m, n, k)) {
    return eval_print(false, 0, 0, "usage: tune-eval --symbol S --bm BM --bn BN --shape m=..,n=..,k=..");
  }
  void *module = nullptr, *fn = nullptr;
  const size_t size = static_cast<size_t>(kh_cli_co_gemm_tune_end - kh_cli_co_gemm_tune);
  if (size == 0 || khrt_module_load_data(&module, kh_cli_co_gemm_tune, size) != 0 ||
      khrt_module_get_function(&fn, module, symbol.c_str()) != 0) {
    return eval_print(false, 0, 0, std::string("load-error: ") + khrt_last_error());
  }
  std::vector<uint64_t> slots;
  std::vector<void *> params;
  auto grid_for = [&](int64_t mm, int64_t nn) {
    return khrt_dim3{static_cast<unsigned>(((mm + bm - 1) / bm) * ((nn + bn - 1) / bn)), 1, 1};
  };
  const khrt_dim3 block{256, 1, 1};

  // Re-verification on the capped shape.
  {
    const int64_t vm = std::min<int64_t>(m, 128), vn = std::min<int64_t>(n, 128), vk = std::min<int64_t>(k, 128);
    std::vector<float> a(vm * vk), b(vk * vn), c(vm * vn);
    fill_uniform(a, 0xA5A5u);
    fill_uniform(b, 0x5A5Au);
    void *dA = nullptr, *dB = nullptr, *dC = nullptr;
    if (khrt_malloc(&dA, a.size() * 4) || khrt_malloc(&dB, b.size() * 4) || khrt_malloc(&dC, c.size() * 4)) {
      return eval_print(false, 0, 0, "reverify: allocation failed");
    }
    khrt_memcpy_h2d(dA, a.data(), a.size() * 4);
    khrt_memcpy_h2d(dB, b.data(), b.size() * 4);
    fill_args(dA, dB, dC, vm, vn, vk, slots, params);
    if (khrt_launch_raw(fn, grid_for(vm, vn), block, 0, nullptr, params.data()) != 0 ||
        khrt_device_synchronize() != 0) {
      return eval_print(false, 0, 0, std::string("reverify: launch failed: ") + khrt_last_error());
    }
    khrt_memcpy_d2h(c.data(), dC, c.size() * 4);
    double num = 0.0, den = 0.0;
    for (int64_t i = 0; i < vm; ++i)
      for (int64_t j = 0; j < vn; ++j) {
        double r = 0.0;
        for (int64_t q = 0; q < vk; ++q) r += static_cast<double>(a[i * vk + q]) * b[q * vn + j];
        num += (c[i * vn + j] - r) * (c[i * vn + j] - r);
        den += r * r;
      }
    khrt_free(dA);
    khrt_free(dB);
    khrt_free(dC);
    const double rel = std::sqrt(num / std::max(den, 1e-300));
    if (!(rel <= 1e-5)) {
      char buf[96];
      std::snprintf(buf, sizeof buf, "reverify: FAIL rel-frobenius=%.3e", rel);
      return eval_print(false, 0, 0, buf);
    }
  }

  // Timing at the tuning shape: warmup 3, median of 10.
  void *dA = nullptr, *dB = nullptr, *dC = nullptr;
  if (khrt_malloc(&dA, m * k * 4) || khrt_malloc(&dB, k * n * 4) || khrt_malloc(&dC, m * n * 4)) {
    return eval_print(false, 0, 0, "allocation failed at the tuning shape");
  }
  khrt_fill_f32(dA, 1.0f, static_cast<size_t>(m * k), nullptr);
  khrt_fill_f32(dB, 0.5f, static_cast<size_t>(k * n), nullptr);
  fill_args(dA, dB, dC, m, n, k, slots, params);
  for (int i = 0; i < 3; ++i) khrt_launch_raw(fn, grid_for(m, n), block, 0, nullptr, params.data());
  khrt_device_synchronize();
  void *e0 = nullptr, *e1 = nullptr;
  khrt_event_create(&e0);
  khrt_event_create(&e1);
  std::vector<double> ms;
  for (int i = 0; i < 10; ++i) {
    khrt_event_record(e0, nullptr);
    khrt_launch_raw(fn, grid_for(m, n), block, 0, nullptr, params.data());
    khrt_event_record(e1, nullptr);
    khrt_event_synchronize(e1);
    float t = 0.0f;
    khrt_event_elapsed_ms(&t, e0, e1);
    ms.push_back(t);
  }
  std::sort(ms.begin(), ms.end());
  const double med = 0.5 * (ms[4] + ms[5]);
  khrt_free(dA);
  khrt_free(dB);
  khrt_free(dC);
  return eval_print(true, med, 2.0 * m * n * k / (med * 1e6), "ok");
}

int run_tune(int argc, char **argv) {
  std::string kernel = "gemm", shape, out, target = "amdgcn-gfx950", cache = "build/tune-cache.json", v;
  int max_candidates = 80, timeout_s = 30;
  for (int i = 2; i < argc; ++i) {
    const std::string arg = argv[i];
    if (arg == "--help" || arg == "-h") {
      usage_tune(std::cout);
      return 0;
    } else if (take(argc, argv, i, arg, "--kernel", v)) {
      kernel = v;
    } else if (take(argc, argv, i, arg, "--shape", v)) {
      shape = v;
    } else if (take(argc, argv, i, arg, "--out", v)) {
      out = v;
    } else if (take(argc, argv, i, arg, "--target", v)) {
      target = v;
    } else if (take(argc, argv, i, arg, "--cache", v)) {
      cache = v;
    } else if (take(argc, argv, i, arg, "--max-candidates", v)) {
      max_candidates = std::atoi(v.c_str());
      if (max_candidates < 1 || max_candidates > 80) {
        std::cerr << "error: --max-candidates must be an integer in [1,80]\n";
        return 2;
      }
    } else if (take(argc, argv, i, arg, "--timeout", v)) {
      timeout_s = std::atoi(v.c_str());
      if (timeout_s < 1 || timeout_s > 3600) {
        std::cerr << "error: --timeout must be an integer in [1,3600]\n";
        return 2;
      }
    } else {
      std::cerr << "error: unknown flag '" << arg << "' for tune\n";
      return 2;
    }
  }
  int64_t m, n, k;
  if (shape.empty() || out.empty()) {
    std::cerr << "error: tune requires --shape m=...,n=...,k=... and --out <dir>\n";
    return 2;
  }
  if (kernel != "gemm") {
    std::cerr << "error: tune currently supports only the 'gemm' kernel (the config space is GEMM-shaped)\n";
    return 1;
  }
  if (!parse_mnk(shape, m, n, k)) {
    std::cerr << "error: tune requires positive m, n and k in --shape\n";
    return 1;
  }
  if (target != "amdgcn-gfx950") {
    std::cerr << "error: tune requires --target amdgcn-gfx950 (the local execution target)\n";
    return 1;
  }
  const std::string exe = self_exe();
  int status = 0;
  bool timed_out = false;
  const std::string probe = run_child({exe, "tune-eval", "--probe"}, timeout_s, status, timed_out);
  const auto dev = probe.find("DEVICE ");
  if (dev == std::string::npos) {
    std::cerr << "skip: no HIP device available\n";
    return 77;
  }
  const std::string device = probe.substr(dev + 7, probe.find('\n', dev) - dev - 7);
  const std::string shape_text = "m=" + std::to_string(m) + ",n=" + std::to_string(n) + ",k=" + std::to_string(k);
  const std::string key = fnv1a_hex(kernel + "|" + shape_text + "|" + device);
  std::cout << "device: " << device << "\ncache-key: " << key << "\n";
  std::error_code ec;
  fs::create_directories(out, ec);
  const fs::path csv_path = fs::path(out) / "tune-results.csv";

  std::string best_symbol, csv_text;
  if (cache_lookup(cache, key, best_symbol, csv_text)) {
    std::cout << "cache-hit\n";
    std::ofstream(csv_path, std::ios::trunc) << csv_text;
    std::cout << "wrote " << csv_path.string() << "\nbest config: " << best_symbol << "\ntune ok (served from cache)\n";
    return 0;
  }

  std::vector<Result> results;
  const int total = static_cast<int>(sizeof(kCandidates) / sizeof(kCandidates[0]));
  for (int i = 0; i < total && i < max_candidates; ++i) {
    const Candidate &c = kCandidates[i];
    Result r;
    r.c = &c;
    const std::string outp = run_child({exe, "tune-eval", "--symbol", c.symbol, "--bm", std::to_string(c.bm()),
                                        "--bn", std::to_string(c.bn()), "--shape", shape_text},
                                       timeout_s, status, timed_out);
    if (timed_out) {
      r.reason = "timeout";
    } else if (WIFSIGNALED(status)) {
      r.reason = "crashed (signal " + std::to_string(WTERMSIG(status)) + ")";
    } else if (field(outp, "accepted").empty()) {
      r.reason = "no result";
    } else {
      r.accepted = field(outp, "accepted") == "1";
      r.ms = std::atof(field(outp, "ms").c_str());
      r.gflops = std::atof(field(outp, "gflops").c_str());
      r.reason = field(outp, "reason");
    }
    std::printf("candidate %-22s %s %.4f ms %.1f GFLOP/s\n", c.symbol, r.accepted ? "ok  " : r.reason.c_str(), r.ms,
                r.gflops);
    std::fflush(stdout);
    results.push_back(r);
  }

  std::ostringstream csv;
  csv << "kernel,shape,bm,bn,bk,waves,unroll,vec,ms_median,accepted,reason,symbol,wave_tile,prio,lds_dma,gflops\n";
  const Result *best = nullptr;
  for (const Result &r : results) {
    csv << kernel << "," << csv_escape(shape_text) << "," << r.c->bm() << "," << r.c->bn() << "," << r.c->bk
        << ",4,1,4," << r.ms << "," << (r.accepted ? "true" : "false") << "," << csv_escape(r.reason) << ","
        << r.c->symbol << "," << r.c->wtm * 32 << "x" << r.c->wtn * 32 << "," << r.c->prio << "," << r.c->dma << ","
        << r.gflops
        << "\n";
    if (r.accepted && (best == nullptr || r.ms < best->ms)) best = &r;
  }
  std::ofstream(csv_path, std::ios::trunc) << csv.str();
  std::cout << "wrote " << csv_path.string() << " (" << results.size() << " rows)\n";
  if (best == nullptr) {
    std::cout << "best config: none (no candidate passed all gates)\ntune ok\n";
    return 0;
  }
  std::printf("best config: %s bm=%d bn=%d bk=%d prio=%d lds_dma=%d ms_median=%.4f (%.1f GFLOP/s)\n",
              best->c->symbol, best->c->bm(), best->c->bn(), best->c->bk, best->c->prio, best->c->dma, best->ms,
              best->gflops);
  cache_store(cache, key, best->c->symbol, csv.str());
  std::cout << "tune ok\n";
  return 0;
}

}  // namespace khcli
