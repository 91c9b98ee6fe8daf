// Device-limits table (with the new gfx950 entry), the pre-launch launch
// verifier, the occupancy report and the verified launch path.
//
// Follows the reference's single-source-of-truth table
// (lib/compiler/device_limits.cpp:45-144), its five verifier rules
// (lib/compiler/launch_verifier.cpp:109-172, diagnostics pinned by
// test/unit/launch_verifier_test.cpp:165-259) and its analytic occupancy
// formulas (lib/compiler/occupancy.cpp:124-221, hand-computed in
// test/unit/occupancy_test.cpp:160-300). The reference splits these over a
// HIP-free compiler library with weak hooks; here one library holds both,
// so the "runtime override" hooks are direct calls guarded by whether a
// device has been initialised.
#include "kernelh/khrt_internal.hpp"

#include <climits>
#include <cstdio>
#include <cstring>
#include <functional>
#include <limits>
#include <mutex>
#include <unordered_map>

namespace {

// ---------------------------------------------------------------------------
// AMD Instinct MI355X (gfx950, CDNA4) - the execution device of this build.
//   lds_bytes_per_workgroup = 163840: 160 KiB LDS per CU on CDNA4; a
//       workgroup may allocate all of it (hipcc accepts 163840 bytes of
//       static LDS for gfx950 and rejects 180224 with "local memory exceeds
//       limit (163840)").
//   wavefront_size = 64: CDNA is wave64 (code-object note
//       .wavefront_size: 64 of every kernel built here).
//   max_threads_per_workgroup = 1024 (hipDeviceProp.maxThreadsPerBlock).
//   max_grid_dim = {2147483647, 65535, 65535}: conservative HIP grid limits;
//       the live device values override them at launch.
//   vram_bytes = 309237645312: 288 GiB of HBM3E (live value overrides).
//   waves_per_cu = 32: 8 wave slots per SIMD x 4 SIMDs
//       (maxThreadsPerMultiProcessor 2048 / 64).
//   reg_file_per_cu = 131072: 4 SIMDs x 512 32-bit registers (256 VGPR + 256
//       AGPR) x 64 lanes, so floor(R / (vgpr x wave)) counts resident waves
//       per CU.
//   cu_count = 0: runtime query (256 on MI355X).
constexpr khrt_device_limits kGfx950 = {163840, 64, 1024, {2147483647, 65535, 65535},
                                        309237645312LL, 32, 131072, 0,
                                        "AMD Instinct MI355X (gfx950)"};

// The reference's two entries, kept so tables and tests written against the
// reference still resolve (device_limits.cpp:45-106).
constexpr khrt_device_limits kGfx1101 = {65536, 32, 1024, {2147483647, 65535, 65535},
                                         17163091968LL, 32, 6144, 0, "AMD Navi 32 (gfx1101)"};
constexpr khrt_device_limits kSm80 = {49152, 32, 1024, {2147483647, 65535, 65535}, 0, 64, 65536, 0,
                                      "NVIDIA A100-class (sm_80, cross)"};

struct TargetEntry {
  const char *token;
  const khrt_device_limits *limits;
};

constexpr TargetEntry kTargets[] = {{"gfx950", &kGfx950}, {"gfx1101", &kGfx1101}, {"sm_80", &kSm80}};

std::string known_targets() {
  std::string s;
  for (const auto &t : kTargets) {
    if (!s.empty()) s += ", ";
    s += t.token;
  }
  return s;
}

const char *name_of(const khrt_device_limits &l) { return l.name != nullptr ? l.name : "(unknown device)"; }

bool g_have_live = false;
khrt_device_limits g_live;
std::mutex g_live_mu;

// Vendor occupancy API for a loaded function: blocks per CU, -1 if
// unavailable (the reference's query_occupancy_max_blocks_runtime hook,
// lib/runtime/query_occupancy.cpp).
// Answers are cached per (function, block, shared): the query is a
// few microseconds of host time, paid on every verified launch otherwise.
// The cache is dropped whenever a module is unloaded (function handles of
// an unloaded module may be reused).
struct OccKey {
  void *function;
  int block;
  size_t shared;
  bool operator==(const OccKey &o) const { return function == o.function && block == o.block && shared == o.shared; }
};
struct OccKeyHash {
  size_t operator()(const OccKey &k) const {
    return std::hash<void *>()(k.function) ^ (size_t(k.block) << 20) ^ (k.shared << 1);
  }
};
std::mutex g_occ_mu;
std::unordered_map<OccKey, int, OccKeyHash> g_occ;

int occupancy_blocks(void *function, int block, size_t shared) {
  if (function == nullptr || block <= 0) return -1;
  const OccKey key{function, block, shared};
  {
    std::lock_guard<std::mutex> lock(g_occ_mu);
    auto it = g_occ.find(key);
    if (it != g_occ.end()) return it->second;
  }
  int blocks = 0;
  const hipError_t e = hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(
      &blocks, static_cast<hipFunction_t>(function), block, shared);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    blocks = -1;
  }
  std::lock_guard<std::mutex> lock(g_occ_mu);
  g_occ[key] = blocks;
  return blocks;
}

// The kernel's own workgroup-size bound (its __launch_bounds__ /
// max_flat_workgroup_size), cached per function handle until a module is
// unloaded (a later module's function can reuse the address; see
// clear_occupancy_cache); -1 when unknown. A launch above it is undefined for
// the compiled code (register allocation, wave indexing), not merely slow.
std::mutex g_fmax_mu;
std::unordered_map<void *, int> g_fmax;

int function_max_threads(void *function) {
  {
    std::lock_guard<std::mutex> lock(g_fmax_mu);
    auto it = g_fmax.find(function);
    if (it != g_fmax.end()) return it->second;
  }
  int v = -1;
  if (hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, static_cast<hipFunction_t>(function)) !=
      hipSuccess) {
    (void)hipGetLastError();
    v = -1;
  }
  std::lock_guard<std::mutex> lock(g_fmax_mu);
  g_fmax[function] = v;
  return v;
}

std::string analytic_occupancy_violation(const khrt_launch_config &c, const khrt_device_limits &l) {
  if (l.waves_per_cu <= 0 || l.wavefront_size <= 0 || c.threads_per_workgroup <= 0) return "";
  const long need = (static_cast<long>(c.threads_per_workgroup) + l.wavefront_size - 1) / l.wavefront_size;
  if (need > l.waves_per_cu) {
    return "occupancy would be 0 on target '" + std::string(name_of(l)) + "': threads per workgroup " +
           std::to_string(c.threads_per_workgroup) + " needs " + std::to_string(need) +
           " wavefronts, exceeding the target's per-CU budget of " + std::to_string(l.waves_per_cu) +
           " wavefronts (waves_per_cu * wavefront_size)";
  }
  return "";
}

std::string occupancy_violation(const khrt_launch_config &c, const khrt_device_limits &l, void *function) {
  if (function != nullptr && c.threads_per_workgroup > 0) {
    const int blocks = occupancy_blocks(function, c.threads_per_workgroup, c.static_shared_bytes);
    if (blocks >= 0) {
      if (blocks == 0) {
        return "occupancy would be 0 on target '" + std::string(name_of(l)) +
               "': hipOccupancyMaxActiveBlocksPerMultiprocessor reported 0 resident blocks per "
               "multiprocessor for threads=" +
               std::to_string(c.threads_per_workgroup) + ", shared=" + std::to_string(c.static_shared_bytes) +
               " bytes";
      }
      return "";
    }
  }
  return analytic_occupancy_violation(c, l);
}

// All violations, one per line; "" when launchable.
std::string verify(const khrt_launch_config &c, const khrt_device_limits &l, void *function) {
  std::vector<std::string> v;
  if (l.lds_bytes_per_workgroup > 0 && c.static_shared_bytes > static_cast<size_t>(l.lds_bytes_per_workgroup)) {
    v.push_back("shared memory " + std::to_string(c.static_shared_bytes) + " bytes exceeds the " +
                std::to_string(l.lds_bytes_per_workgroup) + "-byte LDS limit for target '" + name_of(l) + "'");
  }
  if (l.max_threads_per_workgroup > 0 && c.threads_per_workgroup > l.max_threads_per_workgroup) {
    v.push_back("threads per workgroup " + std::to_string(c.threads_per_workgroup) + " exceeds the max " +
                std::to_string(l.max_threads_per_workgroup));
  }
  if (function != nullptr && c.threads_per_workgroup > 0) {
    const int fmax = function_max_threads(function);
    if (fmax > 0 && c.threads_per_workgroup > fmax) {
      v.push_back("threads per workgroup " + std::to_string(c.threads_per_workgroup) +
                  " exceeds the kernel's own maximum " + std::to_string(fmax) +
                  " (its declared workgroup size bound)");
    }
  }
  if (l.wavefront_size > 1 && c.threads_per_workgroup > 0 && c.threads_per_workgroup % l.wavefront_size != 0) {
    v.push_back("threads per workgroup " + std::to_string(c.threads_per_workgroup) +
                " is not a multiple of the wavefront size " + std::to_string(l.wavefront_size));
  }
  const long g[3] = {c.grid_x, c.grid_y, c.grid_z};
  bool exceeds = false;
  for (int i = 0; i < 3; ++i) {
    if (l.max_grid_dim[i] > 0 && g[i] > l.max_grid_dim[i]) exceeds = true;
  }
  if (exceeds) {
    v.push_back("grid dim (" + std::to_string(g[0]) + "," + std::to_string(g[1]) + "," + std::to_string(g[2]) +
                ") exceeds the target grid limits");
  }
  const std::string occ = occupancy_violation(c, l, function);
  if (!occ.empty()) v.push_back(occ);
  std::string out;
  for (size_t i = 0; i < v.size(); ++i) {
    if (i) out += '\n';
    out += v[i];
  }
  return out;
}

int resolve_live(khrt_device_limits *out) {
  std::lock_guard<std::mutex> lock(g_live_mu);
  if (!g_have_live) {
    khrt_device_info info;
    if (int rc = khrt_get_device_info(&info)) return rc;
    khrt_device_limits l = kGfx950;
    l.lds_bytes_per_workgroup = info.lds_bytes_per_workgroup;
    l.wavefront_size = info.wavefront_size;
    l.max_threads_per_workgroup = info.max_threads_per_workgroup;
    l.cu_count = info.cu_count;
    l.vram_bytes = info.vram_bytes;
    for (int i = 0; i < 3; ++i) {
      if (info.max_grid_dim[i] > 0) l.max_grid_dim[i] = info.max_grid_dim[i];
    }
    g_live = l;
    g_have_live = true;
  }
  *out = g_live;
  return 0;
}

}  // namespace

namespace khrt {

void clear_occupancy_cache() {
  {
    std::lock_guard<std::mutex> lock(g_occ_mu);
    g_occ.clear();
  }
  std::lock_guard<std::mutex> lock(g_fmax_mu);
  g_fmax.clear();
}

int verified_launch(void *function, khrt_dim3 grid, khrt_dim3 block, size_t shared, void *stream, void **params,
                    size_t nparams) {
  if (function == nullptr) return fail(KHRT_E_INVALID, "KernelLaunch::launch: null kernel function handle");
  if (params == nullptr || nparams == 0) return fail(KHRT_E_INVALID, "KernelLaunch::launch: no kernel arguments packed");
  khrt_device_limits limits;
  if (int rc = resolve_live(&limits)) return rc;
  khrt_launch_config c;
  c.grid_x = static_cast<int32_t>(grid.x > INT_MAX ? INT_MAX : grid.x);
  c.grid_y = static_cast<int32_t>(grid.y > INT_MAX ? INT_MAX : grid.y);
  c.grid_z = static_cast<int32_t>(grid.z > INT_MAX ? INT_MAX : grid.z);
  const long long threads = 1LL * block.x * block.y * block.z;
  c.threads_per_workgroup = static_cast<int32_t>(threads > INT_MAX ? INT_MAX : threads);
  c.static_shared_bytes = shared;
  const std::string diag = verify(c, limits, function);
  if (!diag.empty()) return fail(KHRT_E_REFUSED, "KernelLaunch::launch refused: " + diag);
  return khrt_launch_raw(function, grid, block, shared, stream, params);
}

}  // namespace khrt

using namespace khrt;

extern "C" {

int khrt_device_limits_for(const char *target, khrt_device_limits *out) {
  if (out == nullptr) return fail(KHRT_E_INVALID, "khrt_device_limits_for: null output");
  if (target != nullptr) {
    for (const auto &t : kTargets) {
      if (std::strcmp(target, t.token) == 0) {
        *out = *t.limits;
        return 0;
      }
    }
  }
  return fail(KHRT_E_UNKNOWN_TARGET, "unknown device target \"" + std::string(target ? target : "(null)") +
                                         "\"; known targets: " + known_targets());
}

int khrt_device_target_count(void) { return static_cast<int>(sizeof(kTargets) / sizeof(kTargets[0])); }

const char *khrt_device_target_name(int i) {
  if (i < 0 || i >= khrt_device_target_count()) return nullptr;
  return kTargets[i].token;
}

int64_t khrt_query_cu_count(const khrt_device_limits *limits) {
  int count = 0;
  if (hipGetDeviceCount(&count) == hipSuccess && count > 0) {
    int cu = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, current_device()) == hipSuccess && cu > 0) {
      return cu;
    }
  }
  (void)hipGetLastError();
  return limits != nullptr ? limits->cu_count : 0;
}

int khrt_live_limits(khrt_device_limits *out) {
  if (out == nullptr) return fail(KHRT_E_INVALID, "khrt_live_limits: null output");
  return resolve_live(out);
}

int khrt_verify_launch(const khrt_launch_config *config, const khrt_device_limits *limits, void *function,
                       char *diag, size_t cap) {
  if (config == nullptr || limits == nullptr) return fail(KHRT_E_INVALID, "khrt_verify_launch: null argument");
  const std::string d = verify(*config, *limits, function);
  if (diag != nullptr && cap > 0) {
    std::snprintf(diag, cap, "%s", d.c_str());
  }
  if (d.empty()) return 0;
  set_error(d);
  return KHRT_E_REFUSED;
}

int khrt_compute_occupancy(const khrt_occupancy_input *in, const khrt_device_limits *l, void *function,
                          khrt_occupancy_report *r) {
  if (in == nullptr || l == nullptr || r == nullptr) return fail(KHRT_E_INVALID, "khrt_compute_occupancy: null argument");
  std::memset(r, 0, sizeof(*r));
  const bool have_vgpr = in->vgpr_count > 0 && l->reg_file_per_cu > 0 && l->wavefront_size > 0;
  if (have_vgpr) {
    long long w = l->reg_file_per_cu / (1LL * in->vgpr_count * l->wavefront_size);
    if (w < 1) w = 1;
    if (w > l->waves_per_cu) w = l->waves_per_cu;
    r->vgpr_limited_waves = static_cast<int32_t>(w);
  }
  const bool have_lds = in->lds_bytes > 0 && l->lds_bytes_per_workgroup > 0;
  if (have_lds) r->lds_limited_blocks = static_cast<int32_t>(l->lds_bytes_per_workgroup / in->lds_bytes);
  const bool have_threads = in->threads_per_workgroup > 0 && l->max_threads_per_workgroup > 0;
  if (have_threads) r->thread_limited_blocks = l->max_threads_per_workgroup / in->threads_per_workgroup;
  int best = std::numeric_limits<int>::max();
  r->limiter = 0;
  if (have_vgpr) {
    best = r->vgpr_limited_waves;
    r->limiter = 1;
  }
  if (have_lds && r->lds_limited_blocks < best) {
    best = r->lds_limited_blocks;
    r->limiter = 2;
  }
  if (have_threads && r->thread_limited_blocks < best) {
    best = r->thread_limited_blocks;
    r->limiter = 3;
  }
  if (best != std::numeric_limits<int>::max()) {
    r->achieved_waves = best;
    if (l->waves_per_cu > 0) r->theoretical_pct = 100.0 * best / l->waves_per_cu;
  }
  r->measured_blocks = -1;
  if (function != nullptr && in->threads_per_workgroup > 0) {
    const int blocks = occupancy_blocks(function, in->threads_per_workgroup, static_cast<size_t>(in->lds_bytes));
    if (blocks >= 0) {
      r->measured_blocks = blocks;
      const int wpb = l->wavefront_size > 0 ? (in->threads_per_workgroup + l->wavefront_size - 1) / l->wavefront_size : 1;
      if (l->waves_per_cu > 0) {
        const double pct = 100.0 * (1LL * blocks * wpb) / l->waves_per_cu;
        r->measured_pct = pct > 100.0 ? 100.0 : pct;
      }
    } else {
      std::snprintf(r->measured_note, sizeof(r->measured_note),
                    "vendor occupancy API unavailable; measured_pct = 0 (analytic only)");
    }
  } else {
    std::snprintf(r->measured_note, sizeof(r->measured_note),
                  "no loaded kernel function; measured_pct = 0 (analytic only)");
  }
  return 0;
}

}  // extern "C"
