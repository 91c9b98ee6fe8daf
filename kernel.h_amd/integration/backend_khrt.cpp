// backend_khrt.cpp - the reference runtime's Backend (backend.hpp:56-96)
// implemented over the khrt C-ABI, for lib/runtime/ of the reference tree.
// Every virtual maps onto one khrt_* call; a non-zero status becomes the
// reference's Error{code, message} (runtime_error.hpp:24-31) with the
// library's thread-local message.
#include "kernelh/runtime/backend.hpp"
#include "khrt.h"

#include <memory>

namespace kernelh::runtime {
namespace {

template <class T>
Result<T> fail(int rc) {
  const char *m = khrt_last_error();
  return Result<T>(std::unexpect, Error{rc, (m != nullptr && *m != '\0') ? m : khrt_error_string(rc)});
}
Result<void> ok(int rc) {
  if (rc != 0) return fail<void>(rc);
  return {};
}
// Runs `call` (which writes its out-parameter) first, then reads the value.
// Passing the value as a second argument instead would let the compiler read
// it before the call: argument evaluation order is unspecified.
template <class T, class Call>
Result<T> ok_or(Call &&call, const T &v) {
  if (int rc = call()) return fail<T>(rc);
  return v;
}

class KhrtBackend final : public Backend {
 public:
  BackendKind kind() const override { return BackendKind::kHip; }
  Result<void> init_device(int ordinal) override { return ok(khrt_init_device(ordinal)); }
  Result<DeviceInfo> device_info() override {
    khrt_device_info d{};
    if (int rc = khrt_get_device_info(&d)) return fail<DeviceInfo>(rc);
    return DeviceInfo{d.name, static_cast<long>(d.lds_bytes_per_workgroup), d.wavefront_size,
                      d.max_threads_per_workgroup, static_cast<long>(d.cu_count), static_cast<long>(d.vram_bytes)};
  }
  Result<void> device_synchronize() override { return ok(khrt_device_synchronize()); }

  Result<void *> malloc(size_t bytes) override {
    void *p = nullptr;
    return ok_or([&] { return khrt_malloc(&p, bytes); }, p);
  }
  Result<void> free(void *ptr) override { return ok(khrt_free(ptr)); }
  Result<void> memcpy_h2d(void *dst, const void *src, size_t bytes) override {
    return ok(khrt_memcpy_h2d(dst, src, bytes));
  }
  Result<void> memcpy_d2h(void *dst, const void *src, size_t bytes) override {
    return ok(khrt_memcpy_d2h(dst, src, bytes));
  }

  // The interface passes no size (hipModuleLoadData takes none): the
  // image's extent comes from its own ELF headers, and the library then
  // checks every table and section against it and keeps a private copy, so
  // the caller may free the image once this returns.
  Result<void *> module_load_data(const void *image) override {
    size_t size = 0;
    if (int rc = khrt_elf_image_size(image, &size)) return fail<void *>(rc);
    void *m = nullptr;
    return ok_or([&] { return khrt_module_load_data(&m, image, size); }, m);
  }
  Result<void *> module_get_function(void *module, const char *name) override {
    void *f = nullptr;
    return ok_or([&] { return khrt_module_get_function(&f, module, name); }, f);
  }
  Result<void> module_unload(void *module) override { return ok(khrt_module_unload(module)); }

  // Raw launch: no verification (KernelLaunch::launch verifies first, via
  // khrt_kernel_launch).
  Result<void> launch_kernel(void *function, const LaunchDims &grid, const LaunchDims &block, size_t shared_bytes,
                             StreamHandle stream, void *const *params) override {
    return ok(khrt_launch_raw(function, khrt_dim3{grid.x, grid.y, grid.z}, khrt_dim3{block.x, block.y, block.z},
                              shared_bytes, stream, const_cast<void **>(params)));
  }

  Result<EventHandle> event_create() override {
    void *e = nullptr;
    return ok_or<EventHandle>([&] { return khrt_event_create(&e); }, e);
  }
  Result<void> event_record(EventHandle event, StreamHandle stream) override {
    return ok(khrt_event_record(event, stream));
  }
  Result<void> event_synchronize(EventHandle event) override { return ok(khrt_event_synchronize(event)); }
  Result<float> event_elapsed_time(EventHandle start, EventHandle end) override {
    float ms = 0.0f;
    return ok_or([&] { return khrt_event_elapsed_ms(&ms, start, end); }, ms);
  }
  Result<void> event_destroy(EventHandle event) override { return ok(khrt_event_destroy(event)); }
};

}  // namespace

// The factory a caller selects instead of make_hip_backend()
// (backend.hpp:100); declare it beside that one.
std::shared_ptr<Backend> make_khrt_backend() { return std::make_shared<KhrtBackend>(); }

}  // namespace kernelh::runtime
