// kh_scan_noalloc: the scan entry point that allocates nothing.
//
// It has no counterpart in the reference. It is for callers that cannot
// allocate device memory at call time (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc): the caller passes x and y
// only, and the look-back state that kh_scan keeps in the caller's
// totals_hi / totals_lo lives instead in `scratch`, a file-scope device
// array of kScratchBytes per GPU, held until the process ends.
//
// Set-up happens once per device, in khrt_init_device (with that device
// current): the array's device address is taken with hipGetSymbolAddress
// and kept per device, the scan code object is loaded, and the launch shape
// is verified. A set-up failure does not fail khrt_init_device (the other
// entry points do not need it): it is kept per device and returned by every
// kh_scan_noalloc call on that device. The entry point itself only packs its
// parameters on the stack and launches; it calls no allocating routine, and
// refuses a device that was not set up.
//
// The scan's state is self-validating (a signed header and tagged records;
// see the scan kernel), so the zero-filled array needs no clearing before
// the first call and keeps working across calls of any size. All calls on
// one GPU share that GPU's array: two calls that overlap in time on one GPU
// (different streams, no ordering between them) race and give wrong
// results; calls ordered on one stream, or separated by a synchronisation,
// are independent.
#include "kernelh/khrt_internal.hpp"
#include "kh_tiles.h"

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

namespace {

// 512 B for the scan's header (its ticket counters 256 B past its signed
// words, in another cache line), then 16 B per tile of KH_SCAN_TILE
// elements for every tile but the last: 2^31 elements need 139,811 tiles,
// 2.24 MB.
constexpr size_t kScratchBytes = size_t(4) << 20;
constexpr size_t kHeaderBytes = 512;
constexpr int64_t kMaxElements = int64_t(1) << 31;
static_assert(kHeaderBytes + 16 * ((kMaxElements + KH_SCAN_TILE - 1) / KH_SCAN_TILE) <= kScratchBytes,
              "scratch holds the state of the largest accepted scan");

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;

struct DeviceState {
  bool ready = false;
  bool tried = false;        // set-up ran (successfully or not)
  int error_code = 0;        // its failure, returned by every call
  std::string error;
  float *ptr = nullptr;     // device address of this device's `scratch`
  void *function = nullptr;  // `scan` in this device's module
  int64_t resident = 0;      // workgroups of KH_SCAN_THREADS resident at once
};

std::mutex g_mu;
DeviceState g_state[kMaxDevices];

int bad(const std::string &what) { return khrt::fail(KHRT_E_INVALID, "kh_scan_noalloc: " + what); }

}  // namespace

namespace khrt {

namespace {

int setup(int device, DeviceState &s) {
  const hipError_t e = hipGetSymbolAddress(reinterpret_cast<void **>(&s.ptr), HIP_SYMBOL(scratch));
  if (e != hipSuccess) return fail_hip(e, "hipGetSymbolAddress(scratch)");
  if (int rc = khrt_template_function("scan", &s.function)) return rc;
  int per_cu = 0, cus = 0;
  hipError_t q = hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, static_cast<hipFunction_t>(s.function),
                                                                      KH_SCAN_THREADS, 0);
  if (q != hipSuccess) return fail_hip(q, "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(scan)");
  q = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
  if (q != hipSuccess) return fail_hip(q, "hipDeviceGetAttribute(multiprocessor count)");
  s.resident = int64_t(per_cu) * cus;
  if (s.resident <= 0) return fail(KHRT_E_REFUSED, "kh_scan_noalloc set-up: scan has no resident workgroups");
  khrt_device_limits live;
  if (int rc = khrt_live_limits(&live)) return rc;
  khrt_launch_config c{};
  c.threads_per_workgroup = KH_SCAN_THREADS;
  c.grid_x = static_cast<int32_t>(s.resident);
  c.grid_y = c.grid_z = 1;
  char diag[512];
  if (khrt_verify_launch(&c, &live, s.function, diag, sizeof(diag)) != 0) {
    return fail(KHRT_E_REFUSED, std::string("kh_scan_noalloc set-up: scan launch refused: ") + diag);
  }
  s.ready = true;
  return 0;
}

}  // namespace

void noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return;  // such devices are refused at call time
  {
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_state[device].tried) return;
  }
  DeviceState s;
  s.tried = true;
  if (int rc = setup(device, s)) {
    s.ready = false;
    s.error_code = rc;
    s.error = khrt_last_error();
    clear_error();
  }
  std::lock_guard<std::mutex> lock(g_mu);
  g_state[device] = s;
}

}  // namespace khrt

extern "C" int kh_scan_noalloc(const float *x, float *y, int64_t n, void *stream) {
  if (n <= 0) return bad("n must be positive");
  if (n > kMaxElements) {
    return bad("n = " + std::to_string(n) + " exceeds the maximum of 2^31 elements (the look-back state array is " +
               std::to_string(kScratchBytes >> 20) + " MiB per device)");
  }
  if (x == nullptr || y == nullptr) return bad("null buffer");
  const int device = khrt::current_device();
  DeviceState s;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    if (device >= 0 && device < kMaxDevices) s = g_state[device];
  }
  if (!s.ready) {
    if (s.tried) return khrt::fail(s.error_code, "kh_scan_noalloc: set-up on device " + std::to_string(device) +
                                                     " failed: " + s.error);
    return bad("device " + std::to_string(device) +
               " is not set up: call khrt_init_device on it first (the entry point does no set-up of its own)");
  }
  // x, y, y_lo (unused by the kernel: y again), totals_hi (the records),
  // totals_lo (the header): 25 slots on the stack.
  const int64_t header_floats = kHeaderBytes / sizeof(float);
  const int64_t record_floats = (kScratchBytes - kHeaderBytes) / sizeof(float);
  uint64_t slots[25];
  void *params[25];
  const struct {
    const void *ptr;
    int64_t count;
  } args[5] = {{x, n}, {y, n}, {y, n}, {s.ptr + header_floats, record_floats}, {s.ptr, header_floats}};
  for (int i = 0; i < 5; ++i) {
    if (int rc = khrt_pack_memref(slots + 5 * i, 5, args[i].ptr, 1, &args[i].count)) return rc;
  }
  for (int i = 0; i < 25; ++i) params[i] = &slots[i];
  // As kh_scan: at most one resident round of workgroups, each given the
  // same number of tiles.
  const int64_t tiles = (n + KH_SCAN_TILE - 1) / KH_SCAN_TILE;
  const int64_t rounds = (tiles + s.resident - 1) / s.resident;
  const unsigned grid = static_cast<unsigned>((tiles + rounds - 1) / rounds);
  return khrt_launch_raw(s.function, khrt_dim3{grid, 1, 1}, khrt_dim3{KH_SCAN_THREADS, 1, 1}, 0, stream, params);
}
