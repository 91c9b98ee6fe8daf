// `kernelh tune`: GEMM tile autotune over the gfx950 candidates (the
// launcher's own symbols and the tune space of gemm_tune_list.h, both listed
// by the runtime: khrt_gemm_candidate_get), with the reference's evaluator
// contract
// (tools/kernelh/main.cpp:649-673, 1320-1420; lib/compiler/autotuner.cpp):
//   * every candidate is evaluated in a child process with a wall-clock
//     deadline; a hung or crashed candidate is recorded ("timeout",
//     "crashed") and never hangs the run. The parent never initialises HIP:
//     it starts `kernelh tune-eval` children, each of which does;
//   * the child re-verifies the candidate on a small shape (each dimension
//     capped at 128) against an fp64 host product, relative Frobenius
//     <= 1e-5, then times it at the tuning shape: warmup 3, median of 10;
//   * results go to <out>/tune-results.csv (the reference's columns, then
//     symbol, mfma, wave_grid, wave_tile, pipeline, prio, product, gflops)
//     and to a cache file keyed by kernel|shape|device, so a second run with
//     the same key is served from the cache. The runtime's GEMM launcher
//     reads the same file when pointed at it (KHRT_TUNE_CACHE or
//     khrt_set_tune_cache) and then runs the cached best for that shape.
// Differences, each stated in the usage text: the space is a fixed set of
// precompiled instantiations (no per-candidate compilation), small enough
// to evaluate whole, so that is the default (up to --max-candidates); the
// reference's sampled search runs when --sample or --refine-budget is given
// (a fixed-seed sample of the space, then single-step refinement around the
// best accepted candidate, lib/compiler/autotuner.cpp:826-875). The cache key
// is an FNV-1a 64-bit hash (khrt_tune_cache_key).
#include "tune.hpp"

#include "args.hpp"
#include "kernelh/shape_text.hpp"
#include "khrt.h"

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

namespace khcli {
namespace {

namespace fs = std::filesystem;

using Candidate = khrt_gemm_candidate;

std::vector<Candidate> candidates() {
  std::vector<Candidate> out(static_cast<size_t>(khrt_gemm_candidate_count()));
  for (size_t i = 0; i < out.size(); ++i) khrt_gemm_candidate_get(static_cast<int>(i), &out[i]);
  return out;
}

struct Result {
  const Candidate *c = nullptr;
  bool accepted = false;
  double ms = 0.0;
  double gflops = 0.0;
  std::string reason;
};

// m, n and k (all positive, and nothing else) from shape text.
bool parse_mnk(const std::string &text, int64_t &m, int64_t &n, int64_t &k) {
  kernelh::ShapeDims d;
  if (!kernelh::parse_shape_text(text, d) || d.size() != 3 || !d.count("m") || !d.count("n") || !d.count("k")) {
    return false;
  }
  m = d["m"], n = d["n"], k = d["k"];
  return m > 0 && n > 0 && k > 0;
}

// The search order of --sample: the candidate list shuffled by a
// Fisher-Yates pass driven by SplitMix64 from a fixed seed, so a run is
// reproducible.
std::vector<int> sample_order(int total, uint64_t seed) {
  std::vector<int> order(static_cast<size_t>(total));
  for (int i = 0; i < total; ++i) order[static_cast<size_t>(i)] = i;
  auto next = [&seed] {
    uint64_t z = (seed += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  };
  for (int i = total - 1; i > 0; --i) std::swap(order[static_cast<size_t>(i)], order[next() % (i + 1)]);
  return order;
}

// Candidates one design step away from `c`: the same in every field the
// space varies but one (bm, bn, bk, waves, unroll, MFMA shape, pipeline,
// priority, K-split).
bool one_step_apart(const Candidate &a, const Candidate &b) {
  const int diffs = (a.bm != b.bm) + (a.bn != b.bn) + (a.bk != b.bk) + (a.waves != b.waves) +
                    (a.unroll != b.unroll) + (a.mfma != b.mfma) + (std::strcmp(a.pipeline, b.pipeline) != 0) +
                    (a.prio != b.prio) + (a.k_split != b.k_split);
  return diffs == 1;
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
     << "  --max-candidates <n>  cap on evaluated candidates (1.." << khrt_gemm_candidate_count()
     << ", default all)\n"
     << "  --sample <n>          sampled search: n candidates (1..216, default 64) in a\n"
     << "                        fixed pseudo-random order ...\n"
     << "  --refine-budget <n>   ... then up to n (0..80, default 16) candidates one\n"
     << "                        design step from the best; without either flag every\n"
     << "                        candidate is evaluated in list order\n"
     << "  --timeout <seconds>   wall clock per candidate (1..3600, default 30)\n"
     << "  --cache <path>        cache file (default build/tune-cache.json), keyed\n"
     << "                        FNV-1a(kernel|shape|device)\n"
     << "Candidates: the launcher's own gemm symbols, then the gfx950 tune space\n"
     << "(gemm_tune_space.py): MFMA 32x32 or 16x16 wave tiles, 4 or 8 waves, BM/BN in\n"
     << "{64,128,256}, BK in {16,32}, unroll 1 or 2 (register-staged, direct-to-LDS\n"
     << "three stages, or two slabs ahead), MFMA wave priority; vec is 4 (dwordx4)\n"
     << "when k and n are multiples of 4, else 1. The space is precompiled; it is\n"
     << "evaluated whole unless --sample/--refine-budget ask for the sampled search.\n"
     << "Point the runtime at the cache\n"
     << "(KHRT_TUNE_CACHE=<path> or khrt_set_tune_cache) and kh_gemm runs the\n"
     << "cached best for each tuned shape.\n";
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
  std::string symbol, shape;
  bool probe = false;
  for (khcli::ArgCursor a(argc, argv, 2); !a.done();) {
    if (a.value("--symbol", symbol) || a.value("--shape", shape)) continue;
    if (a.flag("--probe")) {
      probe = true;
      continue;
    }
    a.skip();
  }
  int count = 0;
  if (khrt_device_count(&count) != 0 || count < 1 || khrt_init_device(0) != 0) {
    return eval_print(false, 0, 0, "skip: no HIP device");
  }
  if (probe) {
    // The device token and the cache key of --shape, both computed by the
    // runtime, which reads the same cache with the same key.
    char token[512], key[17];
    if (khrt_device_token(token, sizeof token) != 0) return eval_print(false, 0, 0, "skip: no HIP device");
    std::printf("DEVICE %s\n", token);
    if (!shape.empty() && khrt_tune_cache_key("gemm", shape.c_str(), key, sizeof key) == 0) {
      std::printf("KEY %s\n", key);
    }
    return 0;
  }
  int64_t m, n, k;
  if (symbol.empty() || !parse_mnk(shape, m, n, k)) {
    return eval_print(false, 0, 0, "usage: tune-eval --symbol S --shape m=..,n=..,k=..");
  }
  void *fn = nullptr;
  if (khrt_gemm_candidate_function(symbol.c_str(), &fn) != 0) {
    return eval_print(false, 0, 0, std::string("load-error: ") + khrt_last_error());
  }
  std::vector<uint64_t> slots;
  std::vector<void *> params;
  khrt_dim3 block{0, 0, 0};
  auto grid_for = [&](int64_t mm, int64_t nn, int64_t kk) {
    khrt_dim3 g{1, 1, 1};
    khrt_gemm_candidate_geometry(symbol.c_str(), mm, nn, kk, &g, &block);
    return g;
  };
  grid_for(m, n, k);

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
    const khrt_dim3 vgrid = grid_for(vm, vn, vk);
    if (khrt_launch_raw(fn, vgrid, block, 0, nullptr, params.data()) != 0 ||
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
  const khrt_dim3 grid = grid_for(m, n, k);
  for (int i = 0; i < 3; ++i) khrt_launch_raw(fn, grid, block, 0, nullptr, params.data());
  khrt_device_synchronize();
  void *e0 = nullptr, *e1 = nullptr;
  khrt_event_create(&e0);
  khrt_event_create(&e1);
  std::vector<double> ms;
  for (int i = 0; i < 10; ++i) {
    khrt_event_record(e0, nullptr);
    khrt_launch_raw(fn, grid, block, 0, nullptr, params.data());
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
  std::string kernel = "gemm", shape, out, target = "amdgcn-gfx950", cache = "build/tune-cache.json";
  const std::vector<Candidate> space = candidates();
  const int total = static_cast<int>(space.size());
  long max_candidates = total, timeout_s = 30, sample = 64, refine = 16;
  bool searched = false, ok = true;
  for (khcli::ArgCursor a(argc, argv, 2); !a.done() && ok;) {
    if (a.flag("--help") || a.flag("-h")) {
      usage_tune(std::cout);
      return 0;
    }
    if (a.value("--kernel", kernel) || a.value("--shape", shape) || a.value("--out", out) ||
        a.value("--target", target) || a.value("--cache", cache) ||
        a.integer("--max-candidates", 1, total, max_candidates, ok) ||
        a.integer("--timeout", 1, 3600, timeout_s, ok)) {
      continue;
    }
    // The reference's sampled search (main.cpp:710-723): a sample of the
    // space, then single-step refinement around the best.
    if (a.integer("--sample", 1, 216, sample, ok) || a.integer("--refine-budget", 0, 80, refine, ok)) {
      searched = true;
      continue;
    }
    std::cerr << "error: unknown flag '" << a.word() << "' for tune\n";
    return 2;
  }
  if (!ok) return 2;
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
  const std::string shape_text = "m=" + std::to_string(m) + ",n=" + std::to_string(n) + ",k=" + std::to_string(k);
  const std::string probe = run_child({exe, "tune-eval", "--probe", "--shape", shape_text},
                                      static_cast<int>(timeout_s), status, timed_out);
  const auto dev = probe.find("DEVICE ");
  const auto kpos = probe.find("KEY ");
  if (dev == std::string::npos || kpos == std::string::npos) {
    std::cerr << "skip: no HIP device available\n";
    return 77;
  }
  const std::string device = probe.substr(dev + 7, probe.find('\n', dev) - dev - 7);
  const std::string key = probe.substr(kpos + 4, 16);
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
  std::vector<bool> seen(static_cast<size_t>(total), false);
  auto evaluate = [&](int i) {
    const Candidate &c = space[static_cast<size_t>(i)];
    seen[static_cast<size_t>(i)] = true;
    Result r;
    r.c = &c;
    const std::string outp = run_child({exe, "tune-eval", "--symbol", c.symbol, "--shape", shape_text},
                                       static_cast<int>(timeout_s), status, timed_out);
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
    std::printf("candidate %-34s %s %.4f ms %.1f GFLOP/s\n", c.symbol, r.accepted ? "ok  " : r.reason.c_str(), r.ms,
                r.gflops);
    std::fflush(stdout);
    results.push_back(r);
  };
  const int budget = static_cast<int>(max_candidates);
  if (!searched) {
    // Every candidate in list order (the launcher's own symbols first), up
    // to --max-candidates: the space is small enough to evaluate whole.
    for (int i = 0; i < total && i < budget; ++i) evaluate(i);
  } else {
    // --sample candidates in a fixed pseudo-random order, then up to
    // --refine-budget candidates one step from the best accepted one, all
    // within --max-candidates.
    const std::vector<int> order = sample_order(total, 0x6b65726e656c68ull);
    for (int j = 0; j < total && j < sample && static_cast<int>(results.size()) < budget; ++j) evaluate(order[j]);
    const Result *best = nullptr;
    for (const Result &r : results)
      if (r.accepted && (best == nullptr || r.ms < best->ms)) best = &r;
    if (best == nullptr) {
      std::printf("no accepted candidate; skipping refinement\n");
    } else {
      const Candidate centre = *best->c;
      std::vector<int> near;
      for (int i = 0; i < total; ++i)
        if (!seen[static_cast<size_t>(i)] && one_step_apart(space[static_cast<size_t>(i)], centre)) near.push_back(i);
      const int n_refine = std::min<int>({static_cast<int>(refine), static_cast<int>(near.size()),
                                          budget - static_cast<int>(results.size())});
      std::printf("refining around %s with %d neighbour(s)\n", centre.symbol, std::max(n_refine, 0));
      for (int j = 0; j < n_refine; ++j) evaluate(near[static_cast<size_t>(j)]);
    }
  }

  // vec: floats per global load the candidate issues at this shape: float4
  // (dwordx4) when k (and, except for the K-split symbols, which read B a
  // column at a time, n) are multiples of 4, else the guarded scalar path.
  const int vec_tiles = (k % 4 == 0 && n % 4 == 0) ? 4 : 1, vec_ksplit = (k % 4 == 0) ? 4 : 1;
  std::ostringstream csv;
  csv << "kernel,shape,bm,bn,bk,waves,unroll,vec,ms_median,accepted,reason,symbol,mfma,wave_grid,wave_tile,"
         "pipeline,prio,product,gflops\n";
  const Result *best = nullptr;
  for (const Result &r : results) {
    const Candidate &c = *r.c;
    csv << kernel << "," << csv_escape(shape_text) << "," << c.bm << "," << c.bn << "," << c.bk << "," << c.waves
        << "," << c.unroll << "," << (c.k_split ? vec_ksplit : vec_tiles) << "," << r.ms << ","
        << (r.accepted ? "true" : "false") << "," << csv_escape(r.reason) << "," << c.symbol << "," << c.mfma << "x"
        << c.mfma << "," << c.wave_grid_m << "x" << c.wave_grid_n << "," << c.wave_tile_m << "x" << c.wave_tile_n
        << "," << c.pipeline << "," << c.prio << "," << c.product << "," << r.gflops << "\n";
    if (r.accepted && (best == nullptr || r.ms < best->ms)) best = &r;
  }
  std::ofstream(csv_path, std::ios::trunc) << csv.str();
  std::cout << "wrote " << csv_path.string() << " (" << results.size() << " rows)\n";
  if (best == nullptr) {
    std::cout << "best config: none (no candidate passed all gates)\ntune ok\n";
    return 0;
  }
  std::printf("best config: %s bm=%d bn=%d bk=%d waves=%d unroll=%d mfma=%dx%d pipeline=%s prio=%d ms_median=%.4f "
              "(%.1f GFLOP/s)\n",
              best->c->symbol, best->c->bm, best->c->bn, best->c->bk, best->c->waves, best->c->unroll, best->c->mfma,
              best->c->mfma, best->c->pipeline, best->c->prio, best->ms, best->gflops);
  cache_store(cache, key, best->c->symbol, csv.str());
  std::error_code aec;
  const fs::path abs = fs::absolute(cache, aec);
  std::cout << "cache: " << (aec ? cache : abs.string())
            << " (KHRT_TUNE_CACHE=<this path> or khrt_set_tune_cache makes kh_gemm run the best for this shape)\n";
  std::cout << "tune ok\n";
  return 0;
}

}  // namespace khcli
