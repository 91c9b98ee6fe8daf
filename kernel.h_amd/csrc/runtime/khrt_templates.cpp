// The seven kernel.h templates behind the C-ABI: embedded gfx950 code
// objects, the registry, the launcher-owned geometry and one entry point per
// template.
//
// Replaces the reference's name -> template dispatch (lib/dsl/registry.cpp:
// 23-36, lib/dsl/program.cpp:17-51) and the per-kernel launch code its
// callers repeat (bench/harness/kernelh_backend.cpp:205-436,
// test/unit/e2e_*_test.cpp). The reference callers own grid/block; here the
// launcher owns geometry per kernel (the kernels stay correct under the
// reference's geometry too), while the memref argument lists, symbol names
// and the hipModuleLoadData / hipModuleLaunchKernel path are unchanged.
#include "kernelh/khrt_internal.hpp"
#include "gemm_tune_list.h"
#include "kh_tiles.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <mutex>
#include <string>
#include <vector>

// Code objects linked into the library by kh_embed.S (generated at build).
#define KH_DECLARE_CO(name)              \
  extern "C" const unsigned char kh_co_##name[]; \
  extern "C" const unsigned char kh_co_##name##_end[];
KH_DECLARE_CO(vecadd)
KH_DECLARE_CO(fused_gelu)
KH_DECLARE_CO(softmax)
KH_DECLARE_CO(layernorm)
KH_DECLARE_CO(scan)
KH_DECLARE_CO(gemm)
KH_DECLARE_CO(attention)
KH_DECLARE_CO(util)
KH_DECLARE_CO(roofline)
KH_DECLARE_CO(gemm_tune0)
KH_DECLARE_CO(gemm_tune1)
KH_DECLARE_CO(gemm_tune2)
KH_DECLARE_CO(gemm_tune3)
static_assert(KH_GEMM_TUNE_PARTS == 4, "one code object per part of the tune list");

namespace {

struct CodeObject {
  const char *name;
  const unsigned char *begin;
  const unsigned char *end;
};

const CodeObject kCodeObjects[] = {
    {"vecadd", kh_co_vecadd, kh_co_vecadd_end},       {"fused_gelu", kh_co_fused_gelu, kh_co_fused_gelu_end},
    {"softmax", kh_co_softmax, kh_co_softmax_end},    {"layernorm", kh_co_layernorm, kh_co_layernorm_end},
    {"scan", kh_co_scan, kh_co_scan_end},             {"gemm", kh_co_gemm, kh_co_gemm_end},
    {"attention", kh_co_attention, kh_co_attention_end}, {"util", kh_co_util, kh_co_util_end},
    {"roofline", kh_co_roofline, kh_co_roofline_end},
    {"gemm_tune0", kh_co_gemm_tune0, kh_co_gemm_tune0_end},
    {"gemm_tune1", kh_co_gemm_tune1, kh_co_gemm_tune1_end},
    {"gemm_tune2", kh_co_gemm_tune2, kh_co_gemm_tune2_end},
    {"gemm_tune3", kh_co_gemm_tune3, kh_co_gemm_tune3_end},
};

struct KernelResources {
  const char *symbol;
  khrt_kernel_resources r;
};

// Resource notes of every kernel symbol, generated from the code objects.
const KernelResources kResources[] = {
#include "kh_resources.inc"
};

struct Template {
  const char *name;  // template name == kernel symbol
  const char *co;    // code object holding the symbol
};

// Registry order follows the reference's registration (registry.cpp:23-36).
const Template kTemplates[] = {
    {"vecadd", "vecadd"}, {"gemm", "gemm"},         {"softmax", "softmax"},       {"layernorm", "layernorm"},
    {"scan", "scan"},     {"scan_totals", "scan"}, {"fused_gelu", "fused_gelu"}, {"attention", "attention"},
};

const CodeObject *find_co(const char *name) {
  for (const auto &c : kCodeObjects) {
    if (std::strcmp(c.name, name) == 0) return &c;
  }
  return nullptr;
}

const Template *find_template(const char *name) {
  if (name == nullptr) return nullptr;
  for (const auto &t : kTemplates) {
    if (std::strcmp(t.name, name) == 0) return &t;
  }
  return nullptr;
}

std::string registered_list() {
  std::string s;
  for (const auto &t : kTemplates) {
    if (!s.empty()) s += ", ";
    s += t.name;
  }
  return s;
}

int unknown_template(const char *name) {
  return khrt::fail(KHRT_E_INVALID, "unknown kernel '" + std::string(name ? name : "(null)") +
                                        "'; registered kernels: " + registered_list());
}

// Per-device module cache: code object name -> loaded module; symbol ->
// function. Loaded once, kept for the process lifetime.
struct LoadedModule {
  int device;
  std::string co;
  void *module;
};
struct LoadedFunction {
  int device;
  std::string symbol;
  void *function;
};
std::mutex g_mu;
std::vector<LoadedModule> g_modules;
std::vector<LoadedFunction> g_functions;

int get_function(const char *co_name, const char *symbol, void **out) {
  if (int rc = khrt::ensure_device()) return rc;
  const int dev = khrt::current_device();
  std::lock_guard<std::mutex> lock(g_mu);
  for (const auto &f : g_functions) {
    if (f.device == dev && f.symbol == symbol) {
      *out = f.function;
      return 0;
    }
  }
  void *module = nullptr;
  for (const auto &m : g_modules) {
    if (m.device == dev && m.co == co_name) module = m.module;
  }
  if (module == nullptr) {
    const CodeObject *co = find_co(co_name);
    if (co == nullptr) return khrt::fail(KHRT_E_INVALID, std::string("no code object '") + co_name + "'");
    const size_t size = static_cast<size_t>(co->end - co->begin);
    if (size < 64) {
      return khrt::fail(KHRT_E_INVALID, std::string("code object '") + co_name + "' is not part of this build");
    }
    if (int rc = khrt_module_load_data(&module, co->begin, size)) return rc;
    g_modules.push_back({dev, co_name, module});
  }
  void *fn = nullptr;
  if (int rc = khrt_module_get_function(&fn, module, symbol)) return rc;
  g_functions.push_back({dev, symbol, fn});
  *out = fn;
  return 0;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// GEMM candidates: the launcher's own symbols, then the tune space
// (gemm_tune_list.h). Every one takes the template `gemm` arguments and
// computes C = A B for every shape and grid.
enum GemmPipe { kRegs = 1, kDma = 2, kPf2 = 3, kPersistent = 4, kKsplit = 5, kKsplitDeep = 6 };

const char *pipe_name(int pipe) {
  switch (pipe) {
    case kRegs: return "regs";
    case kDma: return "lds-dma";
    case kPf2: return "prefetch2";
    case kPersistent: return "persistent";
    case kKsplit: return "ksplit";
    case kKsplitDeep: return "ksplit-deep";
    default: return "?";
  }
}

struct GemmCandidate {
  const char *symbol;
  const char *co;
  int mfma, wgm, wgn, wtm, wtn, bk, prio, pipe;
  bool product;
  // Persistent symbols: workgroups resident per CU (their LDS and
  // registers), so the launcher's grid is one round of them.
  int per_cu = 2;
  bool ksplit() const { return pipe == kKsplit || pipe == kKsplitDeep; }
  // K-split: each of the 8 waves holds the whole 32x32 tile for its K range.
  int waves() const { return ksplit() ? KH_GEMM_KSPLIT_THREADS / 64 : wgm * wgn; }
  int bm() const { return ksplit() ? KH_GEMM_KSPLIT_BM : mfma * wtm * wgm; }
  int bn() const { return ksplit() ? KH_GEMM_KSPLIT_BN : mfma * wtn * wgn; }
  // Slabs (K-split: batches of 32 k) in flight ahead of the MFMAs.
  int unroll() const { return pipe == kRegs ? 1 : pipe == kKsplitDeep ? 3 : 2; }
};

#define KH_TUNE_CANDIDATE(PART, MF, WGM, WGN, WTM, WTN, BK, PRIO, PIPE, SYM) \
  {#SYM, "gemm_tune" #PART, MF, WGM, WGN, WTM, WTN, BK, PRIO, PIPE, false},
const GemmCandidate kGemmCandidates[] = {
    {"gemm", "gemm", 32, 2, 2, 2, 4, 16, 1, kPersistent, true},
    {"gemm_mid", "gemm", 32, 2, 2, 2, 2, 32, 1, kRegs, true},
    {"gemm_small", "gemm", 16, 4, 2, 1, 2, 32, 1, kPersistent, true},
    {"gemm_small_pf2", "gemm", 16, 2, 2, 2, 2, 32, 1, kPf2, true},
    {"gemm_wide", "gemm", 16, 4, 2, 2, 4, 32, 1, kPersistent, true, 1},
    {"gemm_ksplit", "gemm", 32, 1, 1, 1, 1, 8, 0, kKsplit, true},
    {"gemm_ksplit_deep", "gemm", 32, 1, 1, 1, 1, 8, 0, kKsplitDeep, true},
    KH_GEMM_TUNE_CONFIGS(KH_TUNE_CANDIDATE)};
#undef KH_TUNE_CANDIDATE
constexpr int kGemmCandidateCount = static_cast<int>(sizeof(kGemmCandidates) / sizeof(kGemmCandidates[0]));
static_assert(kGemmCandidateCount == 7 + KH_GEMM_TUNE_COUNT, "candidate table");

const GemmCandidate *find_gemm_candidate(const char *symbol) {
  if (symbol == nullptr) return nullptr;
  for (const auto &c : kGemmCandidates) {
    if (std::strcmp(c.symbol, symbol) == 0) return &c;
  }
  return nullptr;
}

// Grid of a candidate at m x n: one workgroup per tile, except the
// persistent symbols, which get one round of resident workgroups and loop
// (per_cu: two for `gemm` and `gemm_small`, one for `gemm_wide`, whose
// 99 KB of LDS allow no more).
int64_t candidate_grid(const GemmCandidate &c, int64_t m, int64_t n) {
  const int64_t tiles = ceil_div(m, c.bm()) * ceil_div(n, c.bn());
  // The K-split symbols loop over their tiles as well: one workgroup per CU
  // (their registers allow no more) measured better than one per tile
  // beyond a round (768^3 18.0 vs 19.0 us, 512x1024x1024 15.1 vs 15.7).
  if (c.ksplit()) return std::min<int64_t>(tiles, KH_GEMM_CUS);
  if (c.pipe == kPersistent) return std::min<int64_t>(tiles, int64_t(c.per_cu) * KH_GEMM_CUS);
  return tiles;
}

// The tune cache `kernelh tune` writes: one JSON object per line,
// {"key": "<16 hex>", "best": "<symbol>", "csv": "..."}, keyed by FNV-1a 64
// of "gemm|m=..,n=..,k=..|<device token>". The launcher reads it only when a
// path is set (khrt_set_tune_cache, or KHRT_TUNE_CACHE in the environment at
// the first GEMM launch); the file is read once per path.
std::string fnv1a_hex(const std::string &s) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char ch : s) {
    h ^= ch;
    h *= 1099511628211ull;
  }
  char buf[17];
  std::snprintf(buf, sizeof buf, "%016llx", static_cast<unsigned long long>(h));
  return buf;
}

// Asked once per device (hipGetDeviceProperties is not cheap enough to sit
// on every launch).
std::string device_token() {
  static std::mutex mu;
  static std::map<int, std::string> memo;
  if (khrt::ensure_device() != 0) return "";
  const int dev = khrt::current_device();
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = memo.find(dev);
    if (it != memo.end()) return it->second;
  }
  khrt_device_info d{};
  if (khrt_get_device_info(&d) != 0) return "";
  const std::string token = std::string(d.name[0] ? d.name : "AMD Instinct MI355X") + " (" + d.arch + ") cu=" +
                            std::to_string(static_cast<long long>(d.cu_count));
  std::lock_guard<std::mutex> lock(mu);
  memo[dev] = token;
  return token;
}

std::string gemm_shape_text(int64_t m, int64_t n, int64_t k) {
  return "m=" + std::to_string(m) + ",n=" + std::to_string(n) + ",k=" + std::to_string(k);
}

struct TuneCache {
  std::mutex mu;
  bool configured = false;  // khrt_set_tune_cache called, or the environment read
  std::string path;
  bool loaded = false;
  std::map<std::string, std::string> best;  // key -> symbol
};
TuneCache g_tune;

void load_tune_cache_locked() {
  g_tune.best.clear();
  g_tune.loaded = true;
  if (g_tune.path.empty()) return;
  std::ifstream f(g_tune.path);
  std::string line;
  const std::string kk = "{\"key\": \"", kb = "\"best\": \"";
  while (std::getline(f, line)) {
    if (line.rfind(kk, 0) != 0) continue;
    const size_t ke = line.find('"', kk.size());
    const size_t b = line.find(kb);
    if (ke == std::string::npos || b == std::string::npos) continue;
    const size_t be = line.find('"', b + kb.size());
    if (be == std::string::npos) continue;
    g_tune.best[line.substr(kk.size(), ke - kk.size())] = line.substr(b + kb.size(), be - b - kb.size());
  }
}

// The tuned candidate for this GEMM shape, or nullptr (no cache, no entry,
// or an entry naming a symbol this build does not have).
const GemmCandidate *tuned_gemm(int64_t m, int64_t n, int64_t k) {
  std::string key;
  {
    std::lock_guard<std::mutex> lock(g_tune.mu);
    if (!g_tune.configured) {
      const char *env = std::getenv("KHRT_TUNE_CACHE");
      g_tune.path = env != nullptr ? env : "";
      g_tune.configured = true;
      g_tune.loaded = false;
    }
    if (g_tune.path.empty()) return nullptr;
    if (!g_tune.loaded) load_tune_cache_locked();
    if (g_tune.best.empty()) return nullptr;
  }
  const std::string dev = device_token();
  if (dev.empty()) return nullptr;
  key = fnv1a_hex("gemm|" + gemm_shape_text(m, n, k) + "|" + dev);
  std::lock_guard<std::mutex> lock(g_tune.mu);
  auto it = g_tune.best.find(key);
  return it == g_tune.best.end() ? nullptr : find_gemm_candidate(it->second.c_str());
}

// GEMM tile choice: the largest tile whose grid still gives every CU work.
// Rate x busy fraction of the last round of workgroups (kh_tiles.h).
double gemm_score(int64_t tiles, int64_t round, double rate) {
  return rate * static_cast<double>(tiles) / static_cast<double>(ceil_div(tiles, round) * round);
}

const char *heuristic_gemm_symbol(int64_t m, int64_t n, int64_t k) {
  const int64_t tiles64 = ceil_div(m, KH_GEMM_SMALL_BM) * ceil_div(n, KH_GEMM_SMALL_BN);
  if (ceil_div(m, KH_GEMM_KSPLIT_BM) * ceil_div(n, KH_GEMM_KSPLIT_BN) <= KH_GEMM_CUS ||
      (tiles64 < KH_GEMM_CUS && m % KH_GEMM_KSPLIT_BM == 0 && n % KH_GEMM_KSPLIT_BN == 0 &&
       k % KH_GEMM_KSPLIT_INTERIOR_K == 0 && k >= KH_GEMM_KSPLIT_MIN_K)) {
    return k >= KH_GEMM_KSPLIT_DEEP_K ? "gemm_ksplit_deep" : "gemm_ksplit";
  }
  const double big = gemm_score(ceil_div(m, KH_GEMM_BM) * ceil_div(n, KH_GEMM_BN), KH_GEMM_ROUND_BIG,
                                KH_GEMM_RATE_BIG);
  const double mid = gemm_score(ceil_div(m, KH_GEMM_MID_BM) * ceil_div(n, KH_GEMM_MID_BN), KH_GEMM_ROUND_MID,
                                KH_GEMM_RATE_MID);
  const double wide = gemm_score(ceil_div(m, KH_GEMM_WIDE_BM) * ceil_div(n, KH_GEMM_WIDE_BN), KH_GEMM_ROUND_WIDE,
                                 KH_GEMM_RATE_WIDE);
  const double small = gemm_score(ceil_div(m, KH_GEMM_SMALL_BM) * ceil_div(n, KH_GEMM_SMALL_BN),
                                  KH_GEMM_ROUND_SMALL, KH_GEMM_RATE_SMALL);
  if (big >= mid && big >= wide && big >= small) return "gemm";
  if (mid >= wide && mid > small) return "gemm_mid";
  if (wide > small) return "gemm_wide";
  return "gemm_small";
}

// The launcher's GEMM candidate: the tune cache's choice for this shape when
// one is set and names a candidate, the heuristic's otherwise.
const GemmCandidate &gemm_choice(int64_t m, int64_t n, int64_t k) {
  if (const GemmCandidate *t = tuned_gemm(m, n, k)) return *t;
  return *find_gemm_candidate(heuristic_gemm_symbol(m, n, k));
}

unsigned clamp_grid(int64_t g) { return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(g, 1 << 20))); }

using Shape = std::map<std::string, int64_t>;

bool need(const Shape &s, const char *key, int64_t &v) {
  auto it = s.find(key);
  if (it == s.end() || it->second <= 0) return false;
  v = it->second;
  return true;
}

// Launcher-owned geometry per template (see each kernel's header comment).
int geometry(const char *name, const Shape &s, khrt_dim3 &grid, khrt_dim3 &block) {
  block = {256, 1, 1};
  grid = {1, 1, 1};
  int64_t n = 0, rows = 0, cols = 0, m = 0, k = 0, b = 0, h = 0, seq = 0, d = 0;
  const std::string t = name;
  if (t == "vecadd" || t == "fused_gelu") {
    if (!need(s, "n", n)) {
      if (t == "fused_gelu" && need(s, "rows", rows) && need(s, "cols", cols)) {
        n = rows * cols;
      } else {
        return khrt::fail(KHRT_E_INVALID, t + ": shape attribute 'n' is required and must be positive");
      }
    }
    grid.x = clamp_grid(ceil_div(ceil_div(n, 4), 256LL * KH_EW_UNROLL));
  } else if (t == "softmax" || t == "layernorm") {
    if (!need(s, "rows", rows) || !need(s, "cols", cols)) {
      return khrt::fail(KHRT_E_INVALID, t + ": shape attributes 'rows' and 'cols' are required and must be positive");
    }
    grid.x = clamp_grid(ceil_div(rows, 4));
  } else if (t == "scan" || t == "scan_totals") {
    if (!need(s, "n", n)) return khrt::fail(KHRT_E_INVALID, t + ": shape attribute 'n' is required and must be positive");
    if (t == "scan") {
      block.x = n <= KH_SCAN_SMALL_N ? KH_SCAN_SMALL_THREADS : KH_SCAN_THREADS;
      grid.x = clamp_grid(ceil_div(n, int64_t(KH_SCAN_PER_THREAD) * (block.x - 64)));
    } else {
      grid.x = clamp_grid(std::min<int64_t>(ceil_div(ceil_div(n, 256) + 1, 256), 1024));
    }
  } else if (t == "gemm") {
    if (!need(s, "m", m) || !need(s, "n", n) || !need(s, "k", k)) {
      return khrt::fail(KHRT_E_INVALID, "gemm: shape attributes 'm', 'n' and 'k' are required and must be positive");
    }
    const GemmCandidate &c = gemm_choice(m, n, k);
    grid.x = clamp_grid(candidate_grid(c, m, n));
    block.x = static_cast<unsigned>(64 * c.waves());
  } else if (t == "attention") {
    if (!need(s, "batch", b) || !need(s, "heads", h) || !need(s, "seq", seq) || !need(s, "head_dim", d)) {
      return khrt::fail(KHRT_E_INVALID,
                        "attention: shape attributes 'batch', 'heads', 'seq' and 'head_dim' are required and "
                        "must be positive");
    }
    if (d != 64) {
      return khrt::fail(KHRT_E_INVALID, "attention: the kernel is pinned to head_dim = 64 (got head_dim = " +
                                            std::to_string(d) + ")");
    }
    grid = {static_cast<unsigned>(ceil_div(seq, KH_ATTN_BLOCK_Q)), static_cast<unsigned>(h),
            static_cast<unsigned>(b)};
  } else {
    return unknown_template(name);
  }
  return 0;
}

// Symbol the launcher runs for a template at a shape. Every symbol of a
// template takes the same arguments and computes the same result; the
// variants differ in which register paths they compile in (softmax and
// layernorm rows of 1025..4096 floats use the *_wide variant).
const char *launch_symbol(const Template *t, const Shape &s) {
  const std::string n = t->name;
  if (n == "softmax" || n == "layernorm") {
    auto it = s.find("cols");
    if (it != s.end() && it->second > 1024 && it->second <= 4096 && (it->second & 3) == 0) {
      return n == "softmax" ? "softmax_wide" : "layernorm_wide";
    }
  }
  if (n == "gemm") {
    auto m = s.find("m"), nn = s.find("n"), k = s.find("k");
    if (m != s.end() && nn != s.end() && k != s.end()) return gemm_choice(m->second, nn->second, k->second).symbol;
  }
  return t->name;
}

// Code object holding the symbol the launcher runs for a template.
const char *launch_co(const Template *t, const char *symbol) {
  if (std::strcmp(t->name, "gemm") == 0) {
    if (const GemmCandidate *c = find_gemm_candidate(symbol)) return c->co;
  }
  return t->co;
}

// Workgroups of `block` threads of `fn` resident on the whole device at
// once (occupancy per CU x CUs), asked once per function; 0 if unknown.
int64_t resident_workgroups(void *fn, unsigned block) {
  struct Entry {
    void *fn;
    unsigned block;
    int64_t resident;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (const auto &e : cache) {
      if (e.fn == fn && e.block == block) return e.resident;
    }
  }
  int per_cu = 0;
  khrt_device_limits live;
  int64_t resident = 0;
  if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, static_cast<hipFunction_t>(fn),
                                                         static_cast<int>(block), 0) == hipSuccess &&
      per_cu > 0 && khrt_live_limits(&live) == 0 && live.cu_count > 0) {
    resident = int64_t(per_cu) * live.cu_count;
  } else {
    (void)hipGetLastError();
  }
  std::lock_guard<std::mutex> lock(mu);
  cache.push_back({fn, block, resident});
  return resident;
}

// Packs, verifies and launches template `name`.
int launch_template(const char *name, khrt::LaunchArgs &args, const Shape &shape, void *stream) {
  const Template *t = find_template(name);
  if (t == nullptr) return unknown_template(name);
  khrt_dim3 grid, block;
  if (int rc = geometry(name, shape, grid, block)) return rc;
  void *fn = nullptr;
  const char *symbol = launch_symbol(t, shape);
  if (int rc = get_function(launch_co(t, symbol), symbol, &fn)) return rc;
  if (std::strcmp(name, "scan") == 0) {
    // The look-back scan is persistent: one resident wave of workgroups
    // loops over tiles, so launch no more workgroups than fit at once, and
    // as many as give every workgroup the same number of tiles (grid.x is
    // the tile count here): 4370 tiles at n = 2^26 run as 18 full rounds of
    // 243 workgroups, not 17 rounds of 256 and an 18th of 18 tiles, during
    // which HBM idles.
    if (const int64_t resident = resident_workgroups(fn, block.x); resident > 0) {
      const int64_t tiles = grid.x, rounds = ceil_div(tiles, resident);
      grid.x = static_cast<unsigned>(ceil_div(tiles, rounds));
    }
  }
  return khrt::verified_launch(fn, grid, block, 0, stream, args.params(), args.count());
}

int bad(const char *what) { return khrt::fail(KHRT_E_INVALID, what); }

}  // namespace

extern "C" {

int khrt_template_count(void) { return static_cast<int>(sizeof(kTemplates) / sizeof(kTemplates[0])); }

const char *khrt_template_name(int i) {
  if (i < 0 || i >= khrt_template_count()) return nullptr;
  return kTemplates[i].name;
}

int khrt_template_code_object(const char *name, const void **image, size_t *size) {
  if (image == nullptr || size == nullptr) return bad("khrt_template_code_object: null output");
  const Template *t = find_template(name);
  if (t == nullptr) return unknown_template(name);
  const CodeObject *co = find_co(t->co);
  *image = co->begin;
  *size = static_cast<size_t>(co->end - co->begin);
  if (*size < 64) return khrt::fail(KHRT_E_INVALID, std::string("code object for '") + name + "' is not part of this build");
  return 0;
}

int khrt_template_resources(const char *name, khrt_kernel_resources *out) {
  if (out == nullptr) return bad("khrt_template_resources: null output");
  if (name == nullptr) return unknown_template(name);
  for (const auto &r : kResources) {
    if (std::strcmp(r.symbol, name) == 0) {
      *out = r.r;
      return 0;
    }
  }
  return unknown_template(name);
}

int khrt_template_geometry(const char *name, const char *shape, khrt_dim3 *grid, khrt_dim3 *block) {
  if (grid == nullptr || block == nullptr || shape == nullptr) return bad("khrt_template_geometry: null argument");
  if (find_template(name) == nullptr) return unknown_template(name);
  Shape s;
  std::string why;
  if (!kernelh::parse_shape_text(shape, s, &why)) return khrt::fail(KHRT_E_INVALID, "malformed shape: expected " + why);
  return geometry(name, s, *grid, *block);
}

int khrt_template_launch_symbol(const char *name, const char *shape, char *out, size_t cap) {
  if (shape == nullptr || out == nullptr || cap == 0) return bad("khrt_template_launch_symbol: null argument");
  const Template *t = find_template(name);
  if (t == nullptr) return unknown_template(name);
  Shape s;
  std::string why;
  if (!kernelh::parse_shape_text(shape, s, &why)) return khrt::fail(KHRT_E_INVALID, "malformed shape: expected " + why);
  khrt_dim3 grid, block;
  if (int rc = geometry(name, s, grid, block)) return rc;  // the same shape checks as a launch
  const std::string sym = launch_symbol(t, s);
  if (sym.size() + 1 > cap) return bad("khrt_template_launch_symbol: output buffer too small");
  std::memcpy(out, sym.c_str(), sym.size() + 1);
  return 0;
}

int khrt_template_function(const char *name, void **function) {
  if (function == nullptr) return bad("khrt_template_function: null output");
  const Template *t = find_template(name);
  if (t == nullptr) return unknown_template(name);
  return get_function(t->co, t->name, function);
}

int khrt_gemm_candidate_count(void) { return kGemmCandidateCount; }

int khrt_gemm_candidate_get(int i, khrt_gemm_candidate *out) {
  if (out == nullptr) return bad("khrt_gemm_candidate_get: null output");
  if (i < 0 || i >= kGemmCandidateCount) {
    return khrt::fail(KHRT_E_INVALID, "khrt_gemm_candidate_get: index " + std::to_string(i) + " outside [0, " +
                                          std::to_string(kGemmCandidateCount) + ")");
  }
  const GemmCandidate &c = kGemmCandidates[i];
  *out = khrt_gemm_candidate{};
  std::snprintf(out->symbol, sizeof out->symbol, "%s", c.symbol);
  std::snprintf(out->code_object, sizeof out->code_object, "%s", c.co);
  std::snprintf(out->pipeline, sizeof out->pipeline, "%s", pipe_name(c.pipe));
  out->mfma = c.mfma;
  out->waves = c.waves();
  out->wave_grid_m = c.ksplit() ? 1 : c.wgm;
  out->wave_grid_n = c.ksplit() ? 1 : c.wgn;
  out->wave_tile_m = c.ksplit() ? c.bm() : c.mfma * c.wtm;
  out->wave_tile_n = c.ksplit() ? c.bn() : c.mfma * c.wtn;
  out->bm = c.bm();
  out->bn = c.bn();
  out->bk = c.bk;
  out->unroll = c.unroll();
  out->prio = c.prio;
  out->persistent = c.pipe == kPersistent;
  out->k_split = c.ksplit();
  out->product = c.product;
  return 0;
}

int khrt_gemm_candidate_geometry(const char *symbol, int64_t m, int64_t n, int64_t k, khrt_dim3 *grid,
                                 khrt_dim3 *block) {
  (void)k;
  if (grid == nullptr || block == nullptr) return bad("khrt_gemm_candidate_geometry: null output");
  const GemmCandidate *c = find_gemm_candidate(symbol);
  if (c == nullptr) {
    return khrt::fail(KHRT_E_INVALID, std::string("unknown GEMM candidate '") + (symbol ? symbol : "(null)") + "'");
  }
  if (m <= 0 || n <= 0 || k <= 0) return bad("khrt_gemm_candidate_geometry: m, n and k must be positive");
  *grid = khrt_dim3{clamp_grid(candidate_grid(*c, m, n)), 1, 1};
  *block = khrt_dim3{static_cast<unsigned>(64 * c->waves()), 1, 1};
  return 0;
}

int khrt_gemm_candidate_function(const char *symbol, void **function) {
  if (function == nullptr) return bad("khrt_gemm_candidate_function: null output");
  const GemmCandidate *c = find_gemm_candidate(symbol);
  if (c == nullptr) {
    return khrt::fail(KHRT_E_INVALID, std::string("unknown GEMM candidate '") + (symbol ? symbol : "(null)") + "'");
  }
  return get_function(c->co, c->symbol, function);
}

int khrt_set_tune_cache(const char *path) {
  std::lock_guard<std::mutex> lock(g_tune.mu);
  g_tune.configured = true;
  g_tune.path = path != nullptr ? path : "";
  g_tune.loaded = false;
  return 0;
}

int khrt_tune_cache_key(const char *kernel, const char *shape, char *out, size_t cap) {
  if (kernel == nullptr || shape == nullptr || out == nullptr) return bad("khrt_tune_cache_key: null argument");
  if (cap < 17) return bad("khrt_tune_cache_key: output buffer too small (17 bytes needed)");
  const std::string dev = device_token();
  if (dev.empty()) return khrt::fail(KHRT_E_INVALID, "khrt_tune_cache_key: no device");
  const std::string key = fnv1a_hex(std::string(kernel) + "|" + shape + "|" + dev);
  std::memcpy(out, key.c_str(), 17);
  return 0;
}

int khrt_device_token(char *out, size_t cap) {
  if (out == nullptr || cap == 0) return bad("khrt_device_token: null output");
  const std::string dev = device_token();
  if (dev.empty()) return khrt::fail(KHRT_E_INVALID, "khrt_device_token: no device");
  if (dev.size() + 1 > cap) return bad("khrt_device_token: output buffer too small");
  std::memcpy(out, dev.c_str(), dev.size() + 1);
  return 0;
}

int khrt_fill_f32(void *dst, float value, size_t count, void *stream) {
  if (count == 0) return 0;
  if (dst == nullptr) return bad("khrt_fill_f32: null destination");
  void *fn = nullptr;
  if (int rc = get_function("util", "kh_fill_f32", &fn)) return rc;
  khrt::LaunchArgs a;
  a.add_memref(dst, {static_cast<int64_t>(count)});
  a.add_scalar_bytes(&value, sizeof(value));
  const unsigned grid = clamp_grid(ceil_div(static_cast<int64_t>(count), 256 * 4));
  return khrt_launch_raw(fn, khrt_dim3{grid, 1, 1}, khrt_dim3{256, 1, 1}, 0, stream, a.params());
}

int kh_vecadd(const float *a, const float *b, float *c, int64_t n, void *stream) {
  if (n <= 0) return bad("vecadd: n must be positive");
  if (!a || !b || !c) return bad("vecadd: null buffer");
  khrt::LaunchArgs args;
  args.add_memref(a, {n});
  args.add_memref(b, {n});
  args.add_memref(c, {n});
  return launch_template("vecadd", args, {{"n", n}}, stream);
}

int kh_fused_gelu(const float *x, float *tmp, float *out, int64_t n, void *stream) {
  if (n <= 0) return bad("fused_gelu: n must be positive");
  if (!x || !out) return bad("fused_gelu: null buffer");
  khrt::LaunchArgs args;
  args.add_memref(x, {n});
  args.add_memref(tmp, {n});
  args.add_memref(out, {n});
  return launch_template("fused_gelu", args, {{"n", n}}, stream);
}

int kh_softmax(const float *x, float *y, int64_t rows, int64_t cols, void *stream) {
  if (rows <= 0 || cols <= 0) return bad("softmax: rows and cols must be positive");
  if (!x || !y) return bad("softmax: null buffer");
  khrt::LaunchArgs args;
  args.add_memref(x, {rows, cols});
  args.add_memref(y, {rows, cols});
  return launch_template("softmax", args, {{"rows", rows}, {"cols", cols}}, stream);
}

int kh_layernorm(const float *x, const float *gamma, const float *beta, float *y, int64_t rows, int64_t cols,
                 void *stream) {
  if (rows <= 0 || cols <= 0) return bad("layernorm: rows and cols must be positive");
  if (!x || !gamma || !beta || !y) return bad("layernorm: null buffer");
  khrt::LaunchArgs args;
  args.add_memref(x, {rows, cols});
  args.add_memref(gamma, {cols});
  args.add_memref(beta, {cols});
  args.add_memref(y, {rows, cols});
  return launch_template("layernorm", args, {{"rows", rows}, {"cols", cols}}, stream);
}

int kh_scan(const float *x, float *y, float *y_lo, float *totals_hi, float *totals_lo, int64_t n, void *stream) {
  if (n <= 0) return bad("scan: n must be positive");
  if (!x || !y || !totals_hi || !totals_lo) return bad("scan: null buffer");
  // The look-back state (in totals_lo a 32-byte header and 16 bytes of
  // ticket counters, 256 B past it when there is room; in totals_hi 16 B
  // per tile but the last) always fits the reference's T = ceil(n/256)
  // floats of each;
  // the kernel establishes it on first use and keeps it valid across calls.
  const int64_t T = ceil_div(n, 256);
  khrt::LaunchArgs args;
  args.add_memref(x, {n});
  args.add_memref(y, {n});
  args.add_memref(y_lo, {n});
  args.add_memref(totals_hi, {T});
  args.add_memref(totals_lo, {T});
  return launch_template("scan", args, {{"n", n}}, stream);
}

int kh_scan_totals(const float *totals_hi, const float *totals_lo, float *off_hi, float *off_lo, float *off_lo2,
                   float *y, float *y_lo, int64_t n, void *stream) {
  if (n <= 0) return bad("scan_totals: n must be positive");
  if (!totals_hi || !totals_lo || !off_hi || !off_lo || !off_lo2 || !y) return bad("scan_totals: null buffer");
  const int64_t T = ceil_div(n, 256);
  khrt::LaunchArgs args;
  args.add_memref(totals_hi, {T});
  args.add_memref(totals_lo, {T});
  args.add_memref(off_hi, {T});
  args.add_memref(off_lo, {T});
  args.add_memref(off_lo2, {T});
  args.add_memref(y, {n});
  args.add_memref(y_lo, {n});
  return launch_template("scan_totals", args, {{"n", n}}, stream);
}

int kh_gemm(const float *A, const float *B, float *C, int64_t m, int64_t n, int64_t k, void *stream) {
  if (m <= 0 || n <= 0 || k <= 0) return bad("gemm: m, n and k must be positive");
  if (!A || !B || !C) return bad("gemm: null buffer");
  khrt::LaunchArgs args;
  args.add_memref(A, {m, k});
  args.add_memref(B, {k, n});
  args.add_memref(C, {m, n});
  return launch_template("gemm", args, {{"m", m}, {"n", n}, {"k", k}}, stream);
}

int kh_attention(const float *Q, const float *K, const float *V, float *O, int64_t batch, int64_t heads, int64_t seq,
                 int64_t head_dim, void *stream) {
  if (batch <= 0 || heads <= 0 || seq <= 0 || head_dim <= 0) return bad("attention: all extents must be positive");
  if (!Q || !K || !V || !O) return bad("attention: null buffer");
  if (heads > 65535 || batch > 65535) return bad("attention: heads and batch must be <= 65535 (grid y/z)");
  khrt::LaunchArgs args;
  args.add_memref(Q, {batch, heads, seq, head_dim});
  args.add_memref(K, {batch, heads, seq, head_dim});
  args.add_memref(V, {batch, heads, seq, head_dim});
  args.add_memref(O, {batch, heads, seq, head_dim});
  return launch_template("attention", args,
                         {{"batch", batch}, {"heads", heads}, {"seq", seq}, {"head_dim", head_dim}}, stream);
}

// Streaming roofline kernels: 32 workgroups of 256 per CU, grid-strided.
static int launch_stream_roofline(const char *symbol, khrt::LaunchArgs &args, void *stream) {
  void *fn = nullptr;
  if (int rc = get_function("roofline", symbol, &fn)) return rc;
  khrt_device_limits live;
  if (int rc = khrt_live_limits(&live)) return rc;
  const unsigned grid = static_cast<unsigned>(std::max<int64_t>(1, live.cu_count) * 32);
  return khrt::verified_launch(fn, khrt_dim3{grid, 1, 1}, khrt_dim3{256, 1, 1}, 0, stream, args.params(), args.count());
}

static bool vec_ok(const void *p, int64_t n) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0 && n > 0 && (n & 3) == 0;
}

int kh_roofline_triad(const float *a, const float *b, float *c, int64_t n, void *stream) {
  if (!a || !b || !c) return bad("roofline_triad: null buffer");
  if (!vec_ok(a, n) || !vec_ok(b, n) || !vec_ok(c, n)) return bad("roofline_triad: n % 4 == 0 and 16-byte alignment required");
  khrt::LaunchArgs args;
  args.add_memref(a, {n});
  args.add_memref(b, {n});
  args.add_memref(c, {n});
  return launch_stream_roofline("roofline_triad", args, stream);
}

int kh_roofline_copy(const float *src, float *dst, int64_t n, void *stream) {
  if (!src || !dst) return bad("roofline_copy: null buffer");
  if (!vec_ok(src, n) || !vec_ok(dst, n)) return bad("roofline_copy: n % 4 == 0 and 16-byte alignment required");
  khrt::LaunchArgs args;
  args.add_memref(src, {n});
  args.add_memref(dst, {n});
  return launch_stream_roofline("roofline_copy", args, stream);
}

int kh_roofline_mfma(float *out, int64_t blocks, int64_t iters, void *stream) {
  if (!out) return bad("roofline_mfma: null buffer");
  if (blocks <= 0 || blocks > (1 << 20) || iters <= 0) return bad("roofline_mfma: blocks in [1, 2^20], iters > 0");
  void *fn = nullptr;
  if (int rc = get_function("roofline", "roofline_mfma", &fn)) return rc;
  khrt::LaunchArgs args;
  args.add_memref(out, {blocks * 256});
  args.add_scalar_bytes(&iters, sizeof(iters));
  return khrt::verified_launch(fn, khrt_dim3{static_cast<unsigned>(blocks), 1, 1}, khrt_dim3{256, 1, 1}, 0, stream,
                               args.params(), args.count());
}

}  // extern "C"
