// Test-only restatement of the reference's Backend interface
// (include/kernelh/runtime/backend.hpp:22-100): the same names, members and
// virtual signatures, so that a binding compiled against it compiles against
// the reference's header unchanged.
#ifndef KH_RESTATED_BACKEND_HPP
#define KH_RESTATED_BACKEND_HPP

#include "kernelh/runtime/runtime_error.hpp"

#include <cstddef>
#include <memory>
#include <string>

namespace kernelh::runtime {

enum class BackendKind { kHip, kCuda };

struct DeviceInfo {
  std::string name;
  long lds_bytes_per_workgroup = 0;
  int wavefront_size = 0;
  int max_threads_per_workgroup = 0;
  long cu_count = 0;
  long vram_bytes = 0;
};

struct LaunchDims {
  unsigned x = 1, y = 1, z = 1;
};

using EventHandle = void *;
using StreamHandle = void *;

struct KernelFunction {
  void *handle = nullptr;
};

class Backend {
 public:
  virtual ~Backend() = default;
  virtual BackendKind kind() const = 0;
  virtual Result<void> init_device(int device_ordinal) = 0;
  virtual Result<DeviceInfo> device_info() = 0;
  virtual Result<void> device_synchronize() = 0;
  virtual Result<void *> malloc(size_t bytes) = 0;
  virtual Result<void> free(void *ptr) = 0;
  virtual Result<void> memcpy_h2d(void *dst, const void *src, size_t bytes) = 0;
  virtual Result<void> memcpy_d2h(void *dst, const void *src, size_t bytes) = 0;
  virtual Result<void *> module_load_data(const void *image) = 0;
  virtual Result<void *> module_get_function(void *module, const char *name) = 0;
  virtual Result<void> module_unload(void *module) = 0;
  virtual Result<void> launch_kernel(void *function, const LaunchDims &grid, const LaunchDims &block,
                                     size_t shared_bytes, StreamHandle stream, void *const *params) = 0;
  virtual Result<EventHandle> event_create() = 0;
  virtual Result<void> event_record(EventHandle event, StreamHandle stream) = 0;
  virtual Result<void> event_synchronize(EventHandle event) = 0;
  virtual Result<float> event_elapsed_time(EventHandle start, EventHandle end) = 0;
  virtual Result<void> event_destroy(EventHandle event) = 0;
};

}  // namespace kernelh::runtime

#endif
