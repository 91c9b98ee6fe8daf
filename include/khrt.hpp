// khrt.hpp - C++ RAII layer over the khrt C-ABI (khrt.h).
//
// Header-only, C++17. The classes keep the shapes of the reference runtime's
// (include/kernelh/runtime/*.hpp): a factory returning Result<X>, move-only
// ownership of the device resource, release in the destructor. They drop the
// reference's std::shared_ptr<Backend> argument, because the khrt library is
// itself the HIP backend.
//
//   Error, Result<T>     runtime_error.hpp:20-31 (std::expected<T, Error>;
//                        this header carries its own Result, usable before
//                        C++23)
//   DeviceContext        device_context.hpp:15-45
//   Buffer               buffer.hpp:14-48, buffer.cpp:8-64
//   GpuModule            gpu_module.hpp:17-44, gpu_module.cpp:8-64
//   LaunchArgs           descriptor_packing.hpp:27-60
//   KernelLaunch         kernel_launch.hpp:26-65, kernel_launch.cpp:100-132
//   EventTimer           event_timer.hpp:14-44, event_timer.cpp:8-67
//
// The wrapper-level refusals carry the reference's messages with code 1
// (KHRT_E_INVALID); failures inside the library carry its code and
// khrt_last_error(). Nothing here throws except Result::value() on an error.
#ifndef KHRT_HPP
#define KHRT_HPP

#include "khrt.h"

#include <cstddef>
#include <cstdint>
#include <new>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

namespace kh::runtime {

struct Error {
  int code = 0;         // a hipError_t value or a KHRT_E_* code; 0 is success
  std::string message;  // non-empty on failure
  bool is_success() const { return code == 0; }
};

// The error of the last khrt call on this thread that returned `rc`.
inline Error last_error(int rc) {
  const char *m = khrt_last_error();
  return Error{rc, (m != nullptr && *m != '\0') ? std::string(m) : std::string(khrt_error_string(rc))};
}

// Marks an Error as the failure value of a Result (std::unexpected's role).
struct Unexpected {
  Error error;
};
inline Unexpected unexpected(Error e) { return Unexpected{std::move(e)}; }

class BadResultAccess : public std::logic_error {
 public:
  explicit BadResultAccess(const Error &e) : std::logic_error("Result holds an error: " + e.message) {}
};

// A value of T or an Error. T may be move-only (Buffer, GpuModule, ...).
template <class T>
class Result {
 public:
  Result(T value) : ok_(true) { new (&storage_.value) T(std::move(value)); }  // NOLINT: implicit like expected
  Result(Unexpected u) : ok_(false) { new (&storage_.error) Error(std::move(u.error)); }
  Result(Result &&o) noexcept(std::is_nothrow_move_constructible<T>::value) : ok_(o.ok_) {
    if (ok_) new (&storage_.value) T(std::move(o.storage_.value));
    else new (&storage_.error) Error(std::move(o.storage_.error));
  }
  Result(const Result &) = delete;
  Result &operator=(const Result &) = delete;
  Result &operator=(Result &&) = delete;
  ~Result() {
    if (ok_) storage_.value.~T();
    else storage_.error.~Error();
  }

  bool has_value() const { return ok_; }
  explicit operator bool() const { return ok_; }
  T &value() & {
    check();
    return storage_.value;
  }
  const T &value() const & {
    check();
    return storage_.value;
  }
  T &&value() && {
    check();
    return std::move(storage_.value);
  }
  T &operator*() & { return value(); }
  const T &operator*() const & { return value(); }
  T &&operator*() && { return std::move(*this).value(); }
  T *operator->() { return &value(); }
  const T *operator->() const { return &value(); }
  const Error &error() const { return storage_.error; }  // meaningful only when !has_value()

 private:
  void check() const {
    if (!ok_) throw BadResultAccess(storage_.error);
  }
  union Storage {
    Storage() {}
    ~Storage() {}
    T value;
    Error error;
  } storage_;
  bool ok_;
};

template <>
class Result<void> {
 public:
  Result() = default;
  Result(Unexpected u) : ok_(false), error_(std::move(u.error)) {}  // NOLINT
  bool has_value() const { return ok_; }
  explicit operator bool() const { return ok_; }
  void value() const {
    if (!ok_) throw BadResultAccess(error_);
  }
  const Error &error() const { return error_; }

 private:
  bool ok_ = true;
  Error error_;
};

// A khrt status as a Result<void>.
inline Result<void> status(int rc) {
  if (rc == 0) return {};
  return unexpected(last_error(rc));
}

struct LaunchDims {
  unsigned x = 1, y = 1, z = 1;
};
using StreamHandle = void *;
struct KernelFunction {
  void *handle = nullptr;
};

struct DeviceInfo {
  std::string name;
  std::string arch;  // e.g. "gfx950:sramecc+:xnack-"
  long lds_bytes_per_workgroup = 0;
  int wavefront_size = 0;
  int max_threads_per_workgroup = 0;
  long cu_count = 0;
  long vram_bytes = 0;
};

// Selects a device and reads its live properties.
class DeviceContext {
 public:
  static Result<DeviceContext> create(int device_ordinal = 0) {
    if (int rc = khrt_init_device(device_ordinal)) return unexpected(last_error(rc));
    khrt_device_info d{};
    if (int rc = khrt_get_device_info(&d)) return unexpected(last_error(rc));
    return DeviceContext(DeviceInfo{d.name, d.arch, static_cast<long>(d.lds_bytes_per_workgroup), d.wavefront_size,
                                    d.max_threads_per_workgroup, static_cast<long>(d.cu_count),
                                    static_cast<long>(d.vram_bytes)});
  }
  const DeviceInfo &info() const { return info_; }
  const std::string &name() const { return info_.name; }
  long lds_bytes_per_workgroup() const { return info_.lds_bytes_per_workgroup; }
  int wavefront_size() const { return info_.wavefront_size; }
  int max_threads_per_workgroup() const { return info_.max_threads_per_workgroup; }
  long cu_count() const { return info_.cu_count; }
  long vram_bytes() const { return info_.vram_bytes; }
  Result<void> synchronize() const { return status(khrt_device_synchronize()); }

 private:
  explicit DeviceContext(DeviceInfo info) : info_(std::move(info)) {}
  DeviceInfo info_;
};

// One device allocation, freed when the Buffer is destroyed.
class Buffer {
 public:
  static Result<Buffer> allocate(size_t bytes) {
    if (bytes == 0) return unexpected(Error{KHRT_E_INVALID, "Buffer::allocate: zero-size buffer"});
    void *p = nullptr;
    if (int rc = khrt_malloc(&p, bytes)) return unexpected(last_error(rc));
    return Buffer(p, bytes);
  }
  Result<void> copy_from_host(const void *src, size_t bytes) {
    if (bytes > bytes_) return unexpected(Error{KHRT_E_INVALID, "Buffer::copy_from_host: copy size exceeds buffer size"});
    return status(khrt_memcpy_h2d(ptr_, src, bytes));
  }
  Result<void> copy_to_host(void *dst, size_t bytes) const {
    if (bytes > bytes_) return unexpected(Error{KHRT_E_INVALID, "Buffer::copy_to_host: copy size exceeds buffer size"});
    return status(khrt_memcpy_d2h(dst, ptr_, bytes));
  }
  void *device_ptr() { return ptr_; }
  const void *device_ptr() const { return ptr_; }
  size_t size() const { return bytes_; }
  bool valid() const { return ptr_ != nullptr; }

  ~Buffer() { release(); }
  Buffer(const Buffer &) = delete;
  Buffer &operator=(const Buffer &) = delete;
  Buffer(Buffer &&o) noexcept : ptr_(std::exchange(o.ptr_, nullptr)), bytes_(std::exchange(o.bytes_, 0)) {}
  Buffer &operator=(Buffer &&o) noexcept {
    if (this != &o) {
      release();
      ptr_ = std::exchange(o.ptr_, nullptr);
      bytes_ = std::exchange(o.bytes_, 0);
    }
    return *this;
  }

 private:
  Buffer(void *p, size_t bytes) : ptr_(p), bytes_(bytes) {}
  void release() {
    if (ptr_ != nullptr) khrt_free(ptr_);  // best effort: a destructor has no error path
    ptr_ = nullptr;
    bytes_ = 0;
  }
  void *ptr_ = nullptr;
  size_t bytes_ = 0;
};

// A loaded code object, unloaded when the GpuModule is destroyed. The
// library validates the ELF image and keeps its own copy of it, so the
// caller's image may be freed once load() returns.
class GpuModule {
 public:
  static Result<GpuModule> load(const void *image, size_t image_size) {
    if (image == nullptr || image_size == 0) {
      return unexpected(Error{KHRT_E_INVALID, "GpuModule::load: empty module image"});
    }
    void *m = nullptr;
    if (int rc = khrt_module_load_data(&m, image, image_size)) return unexpected(last_error(rc));
    return GpuModule(m);
  }
  // The embedded gfx950 code object of a template ("vecadd", "gemm", ...).
  static Result<GpuModule> load_template(const char *name) {
    const void *image = nullptr;
    size_t size = 0;
    if (int rc = khrt_template_code_object(name, &image, &size)) return unexpected(last_error(rc));
    return load(image, size);
  }
  Result<KernelFunction> get_function(const char *name) const {
    if (module_ == nullptr) {
      return unexpected(Error{KHRT_E_INVALID, "GpuModule::get_function: module already unloaded"});
    }
    void *f = nullptr;
    if (int rc = khrt_module_get_function(&f, module_, name)) return unexpected(last_error(rc));
    return KernelFunction{f};
  }
  Result<void> unload() {
    if (module_ == nullptr) return unexpected(Error{KHRT_E_INVALID, "GpuModule::unload: module already unloaded"});
    return status(khrt_module_unload(std::exchange(module_, nullptr)));
  }

  ~GpuModule() {
    if (module_ != nullptr) khrt_module_unload(module_);
  }
  GpuModule(const GpuModule &) = delete;
  GpuModule &operator=(const GpuModule &) = delete;
  GpuModule(GpuModule &&o) noexcept : module_(std::exchange(o.module_, nullptr)) {}
  GpuModule &operator=(GpuModule &&o) noexcept {
    if (this != &o) {
      if (module_ != nullptr) khrt_module_unload(module_);
      module_ = std::exchange(o.module_, nullptr);
    }
    return *this;
  }

 private:
  explicit GpuModule(void *m) : module_(m) {}
  void *module_ = nullptr;
};

// Kernel parameters as 8-byte slots: each rank-N memref expands to 2N+3
// slots {allocated, aligned, offset 0, sizes[N], row-major strides[N]},
// scalars take one slot each, in the order added.
class LaunchArgs {
 public:
  LaunchArgs() = default;
  // A copy has its own slots; params() then points into those.
  LaunchArgs(const LaunchArgs &o) : slots_(o.slots_) {}
  LaunchArgs &operator=(const LaunchArgs &o) {
    slots_ = o.slots_;
    stale_ = true;
    return *this;
  }
  LaunchArgs(LaunchArgs &&) = default;
  LaunchArgs &operator=(LaunchArgs &&) = default;

  void add_memref(const void *dev_ptr, const std::vector<int64_t> &shape) {
    const size_t n = khrt_memref_slot_count(static_cast<int>(shape.size()));
    const size_t at = slots_.size();
    slots_.resize(at + n);
    khrt_pack_memref(slots_.data() + at, n, dev_ptr, static_cast<int>(shape.size()), shape.data());
    stale_ = true;
  }
  void add_scalar_bytes(const void *value, size_t byte_size) {
    slots_.push_back(0);
    khrt_pack_scalar(&slots_.back(), value, byte_size);
    stale_ = true;
  }
  template <class T>
  void add_scalar(T value) {
    static_assert(std::is_trivially_copyable<T>::value && sizeof(T) <= 8, "a scalar fits one 8-byte slot");
    add_scalar_bytes(&value, sizeof(T));
  }
  size_t param_count() const { return slots_.size(); }
  bool empty() const { return slots_.empty(); }
  const std::vector<uint64_t> &raw_slots() const { return slots_; }
  // params()[i] points at slot i (valid until the next add_*).
  void **params() {
    if (stale_) {
      params_.resize(slots_.size());
      for (size_t i = 0; i < slots_.size(); ++i) params_[i] = &slots_[i];
      stale_ = false;
    }
    return params_.data();
  }

 private:
  std::vector<uint64_t> slots_;
  std::vector<void *> params_;
  bool stale_ = true;
};

// A verified launch: the library checks the configuration against the live
// device's limits (LDS, threads per workgroup, wave multiple, grid extents,
// occupancy) and refuses with "KernelLaunch::launch refused: ..." before
// launching exactly the given kernel.
class KernelLaunch {
 public:
  KernelLaunch &grid(unsigned x, unsigned y = 1, unsigned z = 1) {
    grid_ = {x, y, z};
    return *this;
  }
  KernelLaunch &block(unsigned x, unsigned y = 1, unsigned z = 1) {
    block_ = {x, y, z};
    return *this;
  }
  KernelLaunch &shared_mem_bytes(size_t bytes) {
    shared_ = bytes;
    return *this;
  }
  KernelLaunch &stream(StreamHandle s) {
    stream_ = s;
    return *this;
  }
  KernelLaunch &memref_arg(const void *dev_ptr, const std::vector<int64_t> &shape) {
    args_.add_memref(dev_ptr, shape);
    return *this;
  }
  template <class T>
  KernelLaunch &scalar(T value) {
    args_.add_scalar(value);
    return *this;
  }
  Result<void> launch(KernelFunction function) const {
    if (function.handle == nullptr) {
      return unexpected(Error{KHRT_E_INVALID, "KernelLaunch::launch: null kernel function handle"});
    }
    if (args_.empty()) return unexpected(Error{KHRT_E_INVALID, "KernelLaunch::launch: no kernel arguments packed"});
    return status(khrt_kernel_launch(function.handle, khrt_dim3{grid_.x, grid_.y, grid_.z},
                                     khrt_dim3{block_.x, block_.y, block_.z}, shared_, stream_, args_.params(),
                                     args_.param_count()));
  }
  const LaunchArgs &args() const { return args_; }
  const LaunchDims &grid_dims() const { return grid_; }
  const LaunchDims &block_dims() const { return block_; }
  size_t shared_bytes() const { return shared_; }
  StreamHandle stream_handle() const { return stream_; }

 private:
  LaunchDims grid_{1, 1, 1};
  LaunchDims block_{1, 1, 1};
  size_t shared_ = 0;
  StreamHandle stream_ = nullptr;
  mutable LaunchArgs args_;
};

// A pair of events bracketing work on a stream; destroyed with the timer.
class EventTimer {
 public:
  static Result<EventTimer> create() {
    void *start = nullptr, *end = nullptr;
    if (int rc = khrt_event_create(&start)) return unexpected(last_error(rc));
    if (int rc = khrt_event_create(&end)) {
      Error e = last_error(rc);
      khrt_event_destroy(start);
      return unexpected(std::move(e));
    }
    return EventTimer(start, end);
  }
  Result<void> record_start(StreamHandle s = nullptr) { return status(khrt_event_record(start_, s)); }
  Result<void> record_end(StreamHandle s = nullptr) { return status(khrt_event_record(end_, s)); }
  // Blocks until the end event has completed.
  Result<void> synchronize() const { return status(khrt_event_synchronize(end_)); }
  // Milliseconds between the two events (both complete).
  Result<float> elapsed_milliseconds() const {
    float ms = 0.0f;
    if (int rc = khrt_event_elapsed_ms(&ms, start_, end_)) return unexpected(last_error(rc));
    return ms;
  }

  ~EventTimer() { release(); }
  EventTimer(const EventTimer &) = delete;
  EventTimer &operator=(const EventTimer &) = delete;
  EventTimer(EventTimer &&o) noexcept : start_(std::exchange(o.start_, nullptr)), end_(std::exchange(o.end_, nullptr)) {}
  EventTimer &operator=(EventTimer &&o) noexcept {
    if (this != &o) {
      release();
      start_ = std::exchange(o.start_, nullptr);
      end_ = std::exchange(o.end_, nullptr);
    }
    return *this;
  }

 private:
  EventTimer(void *s, void *e) : start_(s), end_(e) {}
  void release() {
    if (start_ != nullptr) khrt_event_destroy(start_);
    if (end_ != nullptr) khrt_event_destroy(end_);
    start_ = end_ = nullptr;
  }
  void *start_ = nullptr;
  void *end_ = nullptr;
};

}  // namespace kh::runtime

#endif  // KHRT_HPP
