// Checks include/khrt.hpp, the C++ RAII layer over khrt.h.
//
//   khrt_raii_check cpu   error paths and argument packing; needs no device
//   khrt_raii_check gpu   vecadd through DeviceContext / Buffer / GpuModule /
//                         KernelLaunch / EventTimer, bit-exact, plus the
//                         verifier's refusal and the lifecycle errors
//
// Prints one line per check and "raii_check <mode> ok" at the end; exits 1
// at the first failure.
#include "khrt.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

using namespace kh::runtime;

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
bool fails_with(const R &r, int code, const char *msg) {
  return !r.has_value() && r.error().code == code && r.error().message == msg;
}

template <class R>
bool fails(const R &r) {
  return !r.has_value() && r.error().code != 0 && !r.error().message.empty();
}

void cpu_checks() {
  // Result: value, error, and value() on an error.
  Result<int> good(7);
  expect(good.has_value() && *good == 7 && bool(good), "Result<int> holds its value");
  Result<int> bad(unexpected(Error{5, "five"}));
  expect(!bad && bad.error().code == 5 && bad.error().message == "five", "Result<int> holds its error");
  bool threw = false;
  try {
    (void)bad.value();
  } catch (const BadResultAccess &) {
    threw = true;
  }
  expect(threw, "value() on an error throws BadResultAccess");
  expect(status(0).has_value(), "status(0) is success");

  // Wrapper-level refusals carry the reference's messages.
  expect(fails_with(Buffer::allocate(0), KHRT_E_INVALID, "Buffer::allocate: zero-size buffer"),
         "Buffer::allocate(0) refused");
  expect(fails_with(GpuModule::load(nullptr, 0), KHRT_E_INVALID, "GpuModule::load: empty module image"),
         "GpuModule::load(empty) refused");
  const unsigned char junk[128] = {1, 2, 3};
  auto m = GpuModule::load(junk, sizeof(junk));
  expect(fails(m) && m.error().message.find("not an ELF") != std::string::npos, "GpuModule::load(junk) typed error");
  auto t = GpuModule::load_template("matmul");
  expect(fails(t) && t.error().message.find("vecadd") != std::string::npos,
         "GpuModule::load_template(unknown) lists the registered templates");
  KernelLaunch none;
  expect(fails_with(none.launch(KernelFunction{}), KHRT_E_INVALID, "KernelLaunch::launch: null kernel function handle"),
         "launch of a null function refused");
  int dummy = 0;
  expect(fails_with(none.launch(KernelFunction{&dummy}), KHRT_E_INVALID,
                    "KernelLaunch::launch: no kernel arguments packed"),
         "launch with no arguments refused");

  // Packing: a rank-2 memref is 7 slots, scalars one slot each.
  LaunchArgs a;
  const void *p = reinterpret_cast<const void *>(uintptr_t(0x7f0000001000));
  a.add_memref(p, {4, 8});
  a.add_scalar<int32_t>(-3);
  a.add_scalar<float>(1.5f);
  const std::vector<uint64_t> want = {0x7f0000001000, 0x7f0000001000, 0, 4, 8, 8, 1};
  expect(a.param_count() == 9, "rank-2 memref + 2 scalars = 9 slots");
  expect(std::equal(want.begin(), want.end(), a.raw_slots().begin()), "memref slots {ptr, ptr, 0, 4, 8, 8, 1}");
  int32_t i32 = 0;
  float f32 = 0;
  std::memcpy(&i32, &a.raw_slots()[7], 4);
  std::memcpy(&f32, &a.raw_slots()[8], 4);
  expect(i32 == -3 && f32 == 1.5f, "scalars in the low bytes of their slots");
  void **pp = a.params();
  expect(pp[0] == &a.raw_slots()[0] && pp[8] == &a.raw_slots()[8], "params()[i] points at slot i");
  KernelLaunch k;
  k.grid(3, 2).block(256).memref_arg(p, {16});
  expect(k.grid_dims().x == 3 && k.grid_dims().y == 2 && k.grid_dims().z == 1 && k.block_dims().x == 256 &&
             k.args().param_count() == 5 && k.shared_bytes() == 0 && k.stream_handle() == nullptr,
         "KernelLaunch records its configuration");
}

void gpu_checks() {
  auto ctx = DeviceContext::create(0);
  expect(ctx.has_value(), "DeviceContext::create(0)");
  // The marketing name can be empty (containerised boxes report ""), so the
  // check is on the arch string and the wave size.
  expect(ctx->wavefront_size() == 64 && ctx->cu_count() > 0 && ctx->info().arch.rfind("gfx950", 0) == 0,
         "device is gfx950, wave64: '" + ctx->name() + "' " + ctx->info().arch);

  const int64_t n = (1 << 20) + 77;
  std::vector<float> a(n), b(n), c(n, -1.0f);
  for (int64_t i = 0; i < n; ++i) {
    a[i] = float(i % 1009) * 0.25f;
    b[i] = float((i * 7) % 997) * -0.5f;
  }
  auto da = Buffer::allocate(n * 4), db = Buffer::allocate(n * 4), dc = Buffer::allocate(n * 4);
  expect(da && db && dc, "three buffers of n floats");
  expect(da->copy_from_host(a.data(), n * 4).has_value() && db->copy_from_host(b.data(), n * 4).has_value(),
         "copy_from_host");
  expect(fails_with(da->copy_from_host(a.data(), n * 4 + 4), KHRT_E_INVALID,
                    "Buffer::copy_from_host: copy size exceeds buffer size"),
         "oversized copy refused");

  auto mod = GpuModule::load_template("vecadd");
  expect(mod.has_value(), "GpuModule::load_template(vecadd)");
  auto fn = mod->get_function("vecadd");
  expect(fn.has_value(), "get_function(vecadd)");
  expect(fails(mod->get_function("no_such_symbol")), "get_function(unknown) typed error");

  auto timer = EventTimer::create();
  expect(timer.has_value(), "EventTimer::create");
  // The reference's geometry: ceil(n/256) workgroups of 256 threads.
  KernelLaunch k;
  k.grid(unsigned((n + 255) / 256)).block(256);
  k.memref_arg(da->device_ptr(), {n}).memref_arg(db->device_ptr(), {n}).memref_arg(dc->device_ptr(), {n});
  expect(timer->record_start().has_value(), "record_start");
  expect(k.launch(*fn).has_value(), "verified launch of vecadd");
  expect(timer->record_end().has_value() && timer->synchronize().has_value(), "record_end + synchronize");
  auto ms = timer->elapsed_milliseconds();
  expect(ms.has_value() && *ms >= 0.0f, "elapsed_milliseconds = " + std::to_string(ms.has_value() ? *ms : -1));
  expect(dc->copy_to_host(c.data(), n * 4).has_value(), "copy_to_host");
  int64_t bad = 0;
  for (int64_t i = 0; i < n; ++i) bad += (c[i] != a[i] + b[i]);
  expect(bad == 0, "vecadd bit-exact (" + std::to_string(bad) + " differ)");

  // The verifier refuses before anything is launched.
  KernelLaunch wide = k;
  wide.block(2048);
  auto r = wide.launch(*fn);
  expect(!r && r.error().code == KHRT_E_REFUSED && r.error().message.rfind("KernelLaunch::launch refused: ", 0) == 0,
         "2048-thread workgroup refused: " + (r ? std::string() : r.error().message.substr(0, 80)));

  // Ownership moves; a second unload is an error.
  GpuModule moved = std::move(*mod);
  expect(fails_with(mod->get_function("vecadd"), KHRT_E_INVALID, "GpuModule::get_function: module already unloaded"),
         "moved-from module refuses get_function");
  expect(moved.unload().has_value(), "unload");
  expect(fails_with(moved.unload(), KHRT_E_INVALID, "GpuModule::unload: module already unloaded"),
         "second unload refused");
  Buffer keep = std::move(*da);
  expect(keep.valid() && !da->valid() && da->size() == 0, "moved-from buffer is empty");
  expect(ctx->synchronize().has_value(), "device synchronize");
}

}  // namespace

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "cpu";
  if (mode == "cpu") {
    cpu_checks();
  } else if (mode == "gpu") {
    cpu_checks();
    gpu_checks();
  } else {
    std::printf("usage: %s cpu|gpu\n", argv[0]);
    return 2;
  }
  std::printf("raii_check %s ok (%d checks)\n", mode.c_str(), g_checks);
  return 0;
}
