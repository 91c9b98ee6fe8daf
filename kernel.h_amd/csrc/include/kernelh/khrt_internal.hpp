// Internal helpers shared by the khrt translation units (not installed).
#pragma once

#include "khrt.h"

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "kernelh/shape_text.hpp"

namespace khrt {

// Thread-local last-error message (khrt_last_error).
void set_error(const std::string &msg);
void clear_error();

// Records `msg` (plus the HIP error string when code is a hipError_t) and
// returns code, so call sites read `return fail(code, "...")`.
int fail(int code, const std::string &msg);
int fail_hip(hipError_t e, const char *what);

// Ensures a device is current (ordinal 0 unless khrt_init_device chose one).
int ensure_device();
int current_device();

// Verified launch used by both khrt_kernel_launch and the kh_* entry points.
int verified_launch(void *function, khrt_dim3 grid, khrt_dim3 block, size_t shared, void *stream,
                    void **params, size_t nparams);

// Packs memref descriptors into 8-byte slots (LaunchArgs::add_memref).
class LaunchArgs {
 public:
  void add_memref(const void *ptr, std::vector<int64_t> shape);
  void add_scalar_bytes(const void *value, size_t bytes);
  void **params();
  size_t count() const { return slots_.size(); }
  const std::vector<uint64_t> &slots() const { return slots_; }

 private:
  std::vector<uint64_t> slots_;
  std::vector<void *> params_;
};

// "" when b[0..size) is a structurally sound 64-bit AMDGPU ELF image whose
// tables and sections all lie inside it; otherwise the reason.
std::string check_elf_image(const unsigned char *b, size_t size);

// Per-device set-up of the allocation-free scan entry point (its state
// array's address, the scan function, a verified launch shape); run by
// khrt_init_device with the device current. Never fails the caller: a
// failure is kept per device and returned by kh_scan_noalloc there.
void noalloc_setup(int device);

// Drops the cached occupancy answers and kernel workgroup-size bounds
// (called when a module is unloaded: a later module's functions can reuse
// the handles).
void clear_occupancy_cache();

}  // namespace khrt
