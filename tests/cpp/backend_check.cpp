// Checks the reference-side Backend binding (kernel.h_amd/integration/
// backend_khrt.cpp) through the Backend interface only, as the reference's
// runtime classes drive it (buffer.cpp, gpu_module.cpp, event_timer.cpp,
// kernel_launch.cpp), compiled against a restatement of backend.hpp.
//
//   khrt_backend_check cpu   error paths; needs no device
//   khrt_backend_check gpu   vecadd and scan launched raw through
//                            Backend::launch_kernel with the reference's
//                            geometry on uninitialised buffers, bit-exact
//
// Prints one line per check and "backend_check <mode> ok" at the end; exits
// 1 at the first failure.
#include "kernelh/runtime/backend.hpp"
#include "khrt.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

namespace kernelh::runtime {
std::shared_ptr<Backend> make_khrt_backend();
}

using namespace kernelh::runtime;

namespace {

int g_checks = 0;

void expect(bool cond, const std::string &what) {
  ++g_checks;
  if (!cond) {
    std::printf("FAIL: %s\n", what.c_str());
    std::fflush(stdout);
    std::exit(1);
  }
  std::printf("  ok: %s\n", what.c_str());
}

template <class R>
bool fails(const R &r) {
  return !r.has_value() && r.error().code != 0 && !r.error().message.empty();
}

// The embedded code object of a template, as a caller holding only a
// pointer (no size) would pass it to module_load_data.
const void *image_of(const char *name, size_t *size) {
  const void *image = nullptr;
  if (khrt_template_code_object(name, &image, size) != 0) return nullptr;
  return image;
}

void cpu_checks(Backend &be) {
  expect(be.kind() == BackendKind::kHip, "kind() is kHip");
  const unsigned char junk[256] = {0x7f, 'E', 'L', 'F', 1, 1};
  auto m = be.module_load_data(junk);
  expect(fails(m) && m.error().code == KHRT_E_INVALID, "module_load_data(32-bit ELF) typed error: " +
                                                           (m ? std::string() : m.error().message));
  const unsigned char text[64] = "not a code object";
  expect(fails(be.module_load_data(text)), "module_load_data(text) typed error");
  // The image extent read from the ELF headers is the image's own size.
  for (const char *name : {"vecadd", "scan", "gemm", "attention"}) {
    size_t size = 0, extent = 0;
    const void *image = image_of(name, &size);
    const bool read = image != nullptr && khrt_elf_image_size(image, &extent) == 0;
    expect(read && extent == size,
           std::string("ELF extent of ") + name + " = " + std::to_string(extent) + " of " + std::to_string(size));
  }
  expect(fails(be.module_get_function(nullptr, "vecadd")), "module_get_function(null module) typed error");
  expect(fails(be.module_unload(nullptr)), "module_unload(null) typed error");
  expect(fails(be.launch_kernel(nullptr, LaunchDims{}, LaunchDims{}, 0, nullptr, nullptr)),
         "launch_kernel(null function) typed error");
}

// Rank-1 memref descriptors, 5 slots each, in argument order.
struct Params {
  std::vector<uint64_t> slots;
  std::vector<void *> ptrs;
  void memref(const void *p, int64_t n) {
    const size_t at = slots.size();
    slots.resize(at + 5);
    khrt_pack_memref(slots.data() + at, 5, p, 1, &n);
  }
  void *const *get() {
    ptrs.resize(slots.size());
    for (size_t i = 0; i < slots.size(); ++i) ptrs[i] = &slots[i];
    return ptrs.data();
  }
};

void gpu_checks(Backend &be) {
  expect(be.init_device(0).has_value(), "init_device(0)");
  auto info = be.device_info();
  expect(info && info->wavefront_size == 64 && info->cu_count > 0 && info->lds_bytes_per_workgroup >= 65536,
         "device_info: " + (info ? info->name : std::string("?")));

  size_t vsize = 0, ssize = 0;
  const void *vimage = image_of("vecadd", &vsize);
  auto vm = be.module_load_data(vimage);  // no size passed
  expect(vm.has_value(), "module_load_data(vecadd image of " + std::to_string(vsize) + " B)" +
                             (vm ? std::string() : ": " + vm.error().message));
  auto vf = be.module_get_function(*vm, "vecadd");
  expect(vf.has_value(), "module_get_function(vecadd)" + (vf ? std::string() : ": " + vf.error().message));

  const int64_t n = 1000003;
  std::vector<float> a(n), b(n), c(n);
  for (int64_t i = 0; i < n; ++i) {
    a[i] = float(i % 4093) * 0.125f;
    b[i] = float((i * 13) % 2039) * -0.25f;
  }
  auto da = be.malloc(n * 4), db = be.malloc(n * 4), dc = be.malloc(n * 4);
  expect(da && db && dc, "malloc x3");
  expect(be.memcpy_h2d(*da, a.data(), n * 4).has_value() && be.memcpy_h2d(*db, b.data(), n * 4).has_value(),
         "memcpy_h2d");
  Params pv;
  pv.memref(*da, n);
  pv.memref(*db, n);
  pv.memref(*dc, n);
  auto e0 = be.event_create(), e1 = be.event_create();
  expect(e0 && e1, "event_create x2");
  const LaunchDims block{256, 1, 1};
  const LaunchDims vgrid{unsigned((n + 255) / 256), 1, 1};
  expect(be.event_record(*e0, nullptr).has_value(), "event_record(start)");
  expect(be.launch_kernel(*vf, vgrid, block, 0, nullptr, pv.get()).has_value(), "launch_kernel(vecadd)");
  expect(be.event_record(*e1, nullptr).has_value() && be.event_synchronize(*e1).has_value(), "event_record + sync");
  auto ms = be.event_elapsed_time(*e0, *e1);
  expect(ms && *ms >= 0.0f, "event_elapsed_time = " + std::to_string(ms ? *ms : -1.0f) + " ms");
  expect(be.memcpy_d2h(c.data(), *dc, n * 4).has_value(), "memcpy_d2h");
  int64_t bad = 0;
  for (int64_t i = 0; i < n; ++i) bad += (c[i] != a[i] + b[i]);
  expect(bad == 0, "vecadd bit-exact (" + std::to_string(bad) + " differ)");

  // scan on uninitialised totals, twice on the same buffers, reference
  // geometry. Inputs on the 2^-24 grid below 1: every prefix below 2^24 of
  // them is exact in fp64 and the rounded fp32 reference is unique.
  const void *simage = image_of("scan", &ssize);
  auto sm = be.module_load_data(simage);
  expect(sm.has_value(), "module_load_data(scan image)");
  auto sf = be.module_get_function(*sm, "scan");
  expect(sf.has_value(), "module_get_function(scan)");
  const int64_t T = (n + 255) / 256;
  std::vector<float> x(n), y(n), ref(n);
  uint64_t s = 0x9E3779B97F4A7C15ull;
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    x[i] = float(s >> 40) * (1.0f / 16777216.0f);
    acc += x[i];
    ref[i] = float(acc);
  }
  auto dx = be.malloc(n * 4), dy = be.malloc(n * 4), th = be.malloc(T * 4), tl = be.malloc(T * 4);
  expect(dx && dy && th && tl, "malloc scan buffers (totals left uninitialised)");
  expect(be.memcpy_h2d(*dx, x.data(), n * 4).has_value(), "memcpy_h2d(x)");
  for (int call = 0; call < 2; ++call) {
    Params ps;
    ps.memref(*dx, n);
    ps.memref(*dy, n);
    ps.memref(*dy, n);  // y_lo: the kernel does not write it
    ps.memref(*th, T);
    ps.memref(*tl, T);
    expect(be.launch_kernel(*sf, LaunchDims{unsigned(T), 1, 1}, block, 0, nullptr, ps.get()).has_value(),
           "launch_kernel(scan) call " + std::to_string(call));
    expect(be.device_synchronize().has_value(), "device_synchronize");
    expect(be.memcpy_d2h(y.data(), *dy, n * 4).has_value(), "memcpy_d2h(y)");
    int64_t diff = 0;
    for (int64_t i = 0; i < n; ++i) diff += (y[i] != ref[i]);
    expect(diff == 0, "scan bit-exact call " + std::to_string(call) + " (" + std::to_string(diff) + " differ)");
  }

  for (void *p : {*da, *db, *dc, *dx, *dy, *th, *tl}) expect(be.free(p).has_value(), "free");
  expect(be.event_destroy(*e0).has_value() && be.event_destroy(*e1).has_value(), "event_destroy x2");
  expect(be.module_unload(*vm).has_value() && be.module_unload(*sm).has_value(), "module_unload x2");
}

}  // namespace

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "cpu";
  auto be = make_khrt_backend();
  if (mode == "cpu") {
    cpu_checks(*be);
  } else if (mode == "gpu") {
    cpu_checks(*be);
    gpu_checks(*be);
  } else {
    std::printf("usage: %s cpu|gpu\n", argv[0]);
    return 2;
  }
  std::printf("backend_check %s ok (%d checks)\n", mode.c_str(), g_checks);
  return 0;
}
