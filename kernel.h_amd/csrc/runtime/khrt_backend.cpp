// khrt backend: the HIP half of the C-ABI (device, memory, module, raw and
// verified launch, streams, events) plus memref descriptor packing.
//
// Replaces the reference's HipBackend (lib/runtime/backend_hip.cpp:47-245),
// LaunchArgs (lib/runtime/descriptor_packing.cpp:19-60) and
// KernelLaunch::launch (lib/runtime/kernel_launch.cpp:100-132) with one
// C-ABI layer: every entry returns a status code and leaves a thread-local
// message, nothing throws across the boundary.
#include "kernelh/khrt_internal.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <unordered_map>

namespace khrt {

namespace {
thread_local std::string g_error;
int g_device = -1;
std::mutex g_mu;
// Private copy of each loaded module's code object, keyed by module.
std::unordered_map<void *, std::unique_ptr<unsigned char[], void (*)(void *)>> g_images;
}  // namespace

void set_error(const std::string &msg) { g_error = msg.empty() ? std::string("(unspecified error)") : msg; }
void clear_error() { g_error.clear(); }

int fail(int code, const std::string &msg) {
  set_error(msg);
  return code == 0 ? KHRT_E_INVALID : code;
}

int fail_hip(hipError_t e, const char *what) {
  return fail(static_cast<int>(e), std::string(what) + ": " + hipGetErrorString(e) + " (hipError_t " +
                                       std::to_string(static_cast<int>(e)) + ")");
}

int ensure_device() {
  if (g_device >= 0) return 0;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0) {
    return fail(KHRT_E_NO_DEVICE, std::string("no HIP device available: ") + hipGetErrorString(e));
  }
  e = hipSetDevice(0);
  if (e != hipSuccess) return fail_hip(e, "hipSetDevice(0)");
  g_device = 0;
  return 0;
}

int current_device() { return g_device < 0 ? 0 : g_device; }

void LaunchArgs::add_memref(const void *ptr, std::vector<int64_t> shape) {
  const uint64_t p = static_cast<uint64_t>(reinterpret_cast<uintptr_t>(ptr));
  slots_.push_back(p);  // allocated
  slots_.push_back(p);  // aligned
  slots_.push_back(0);  // offset
  for (int64_t d : shape) slots_.push_back(static_cast<uint64_t>(d));
  std::vector<uint64_t> strides(shape.size());
  int64_t s = 1;
  for (int i = static_cast<int>(shape.size()) - 1; i >= 0; --i) {
    strides[static_cast<size_t>(i)] = static_cast<uint64_t>(s);
    s *= shape[static_cast<size_t>(i)];
  }
  slots_.insert(slots_.end(), strides.begin(), strides.end());
}

void LaunchArgs::add_scalar_bytes(const void *value, size_t bytes) {
  uint64_t w = 0;
  if (value != nullptr && bytes > 0) std::memcpy(&w, value, bytes < 8 ? bytes : 8);
  slots_.push_back(w);
}

void **LaunchArgs::params() {
  params_.clear();
  params_.reserve(slots_.size());
  for (uint64_t &s : slots_) params_.push_back(&s);
  return params_.data();
}

// Structural check of a 64-bit little-endian AMDGPU ELF image of `size`
// bytes: header fields, and program headers, section headers and every
// section with file contents inside the image. Returns "" when sound.
std::string check_elf_image(const unsigned char *b, size_t size) {
  auto rd16 = [&](size_t off) { uint16_t v; std::memcpy(&v, b + off, 2); return v; };
  auto rd32 = [&](size_t off) { uint32_t v; std::memcpy(&v, b + off, 4); return v; };
  auto rd64 = [&](size_t off) { uint64_t v; std::memcpy(&v, b + off, 8); return v; };
  auto inside = [&](uint64_t off, uint64_t len) { return off <= size && len <= size - off; };
  if (b[4] != 2 || b[5] != 1) return "image is not a 64-bit little-endian ELF";
  if (rd16(18) != 0xE0) return "image is not an AMDGPU code object (e_machine " + std::to_string(rd16(18)) + ")";
  const uint64_t phoff = rd64(32), shoff = rd64(40);
  const uint16_t phentsize = rd16(54), phnum = rd16(56), shentsize = rd16(58), shnum = rd16(60);
  if (phnum > 0 && (phentsize < 56 || !inside(phoff, uint64_t(phentsize) * phnum))) {
    return "program header table lies outside the image (truncated?)";
  }
  if (shnum > 0 && (shentsize < 64 || !inside(shoff, uint64_t(shentsize) * shnum))) {
    return "section header table lies outside the image (truncated?)";
  }
  for (uint16_t i = 0; i < phnum; ++i) {
    const size_t p = phoff + size_t(i) * phentsize;
    if (!inside(rd64(p + 8), rd64(p + 32))) return "segment " + std::to_string(i) + " lies outside the image";
  }
  for (uint16_t i = 0; i < shnum; ++i) {
    const size_t s = shoff + size_t(i) * shentsize;
    const uint32_t type = rd32(s + 4);
    if (type != 8 /* SHT_NOBITS */ && type != 0 && !inside(rd64(s + 24), rd64(s + 32))) {
      return "section " + std::to_string(i) + " lies outside the image";
    }
  }
  return "";
}

}  // namespace khrt

using namespace khrt;

extern "C" {

const char *khrt_last_error(void) { return g_error.c_str(); }

const char *khrt_error_string(int code) {
  switch (code) {
    case KHRT_OK: return "success";
    case KHRT_E_INVALID: return "invalid argument";
    case KHRT_E_REFUSED: return "launch refused by the pre-launch verifier";
    case KHRT_E_UNKNOWN_TARGET: return "unknown device target";
    case KHRT_E_NO_DEVICE: return "no HIP device available";
    case KHRT_E_SKIP: return "skipped";
    default: return hipGetErrorString(static_cast<hipError_t>(code));
  }
}

const char *khrt_version(void) { return "khrt 0.1 (gfx950)"; }

int khrt_device_count(int *count) {
  if (count == nullptr) return fail(KHRT_E_INVALID, "khrt_device_count: null output");
  int c = 0;
  const hipError_t e = hipGetDeviceCount(&c);
  if (e != hipSuccess) {
    *count = 0;
    return fail(KHRT_E_NO_DEVICE, std::string("hipGetDeviceCount: ") + hipGetErrorString(e));
  }
  *count = c;
  return 0;
}

int khrt_init_device(int ordinal) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0) {
    return fail(KHRT_E_NO_DEVICE, std::string("no HIP device available: ") + hipGetErrorString(e));
  }
  if (ordinal < 0 || ordinal >= count) {
    return fail(KHRT_E_INVALID, "khrt_init_device: ordinal " + std::to_string(ordinal) + " out of range [0, " +
                                    std::to_string(count) + ")");
  }
  e = hipSetDevice(ordinal);
  if (e != hipSuccess) return fail_hip(e, "hipSetDevice");
  g_device = ordinal;
  // Optional: a failure here is kept for kh_scan_noalloc and fails nothing else.
  noalloc_setup(ordinal);
  return 0;
}

int khrt_get_device_info(khrt_device_info *out) {
  if (out == nullptr) return fail(KHRT_E_INVALID, "khrt_get_device_info: null output");
  if (int rc = ensure_device()) return rc;
  hipDeviceProp_t p;
  const hipError_t e = hipGetDeviceProperties(&p, g_device);
  if (e != hipSuccess) return fail_hip(e, "hipGetDeviceProperties");
  std::memset(out, 0, sizeof(*out));
  std::snprintf(out->name, sizeof(out->name), "%s", p.name);
  std::snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
  out->lds_bytes_per_workgroup = static_cast<int64_t>(p.sharedMemPerBlock);
  out->wavefront_size = p.warpSize;
  out->max_threads_per_workgroup = p.maxThreadsPerBlock;
  out->cu_count = p.multiProcessorCount;
  out->vram_bytes = static_cast<int64_t>(p.totalGlobalMem);
  for (int i = 0; i < 3; ++i) out->max_grid_dim[i] = p.maxGridSize[i];
  out->clock_khz = p.clockRate;
  out->memory_clock_khz = p.memoryClockRate;
  out->memory_bus_width = p.memoryBusWidth;
  out->l2_bytes = p.l2CacheSize;
  return 0;
}

int khrt_device_synchronize(void) {
  if (int rc = ensure_device()) return rc;
  const hipError_t e = hipDeviceSynchronize();
  return e == hipSuccess ? 0 : fail_hip(e, "hipDeviceSynchronize");
}

int khrt_malloc(void **out, size_t bytes) {
  if (out == nullptr) return fail(KHRT_E_INVALID, "khrt_malloc: null output");
  *out = nullptr;
  if (int rc = ensure_device()) return rc;
  const hipError_t e = hipMalloc(out, bytes == 0 ? 1 : bytes);
  return e == hipSuccess ? 0 : fail_hip(e, "hipMalloc");
}

int khrt_free(void *ptr) {
  if (ptr == nullptr) return 0;
  const hipError_t e = hipFree(ptr);
  return e == hipSuccess ? 0 : fail_hip(e, "hipFree");
}

int khrt_memcpy_h2d(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return 0;
  if (dst == nullptr || src == nullptr) return fail(KHRT_E_INVALID, "khrt_memcpy_h2d: null pointer");
  const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
  return e == hipSuccess ? 0 : fail_hip(e, "hipMemcpy H2D");
}

int khrt_memcpy_d2h(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return 0;
  if (dst == nullptr || src == nullptr) return fail(KHRT_E_INVALID, "khrt_memcpy_d2h: null pointer");
  const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
  return e == hipSuccess ? 0 : fail_hip(e, "hipMemcpy D2H");
}

int khrt_memcpy_d2d(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return 0;
  if (dst == nullptr || src == nullptr) return fail(KHRT_E_INVALID, "khrt_memcpy_d2d: null pointer");
  const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice);
  return e == hipSuccess ? 0 : fail_hip(e, "hipMemcpy D2D");
}

int khrt_module_load_data(void **module, const void *image, size_t size) {
  if (module == nullptr || image == nullptr || size < 64) {
    return fail(KHRT_E_INVALID, "khrt_module_load_data: null or truncated image");
  }
  *module = nullptr;
  const unsigned char *b = static_cast<const unsigned char *>(image);
  if (!(b[0] == 0x7f && b[1] == 'E' && b[2] == 'L' && b[3] == 'F')) {
    return fail(KHRT_E_INVALID, "khrt_module_load_data: image is not an ELF code object");
  }
  // hipModuleLoadData takes no size: a truncated image would be read past
  // its end by the runtime. Check every table and section the loader will
  // touch lies inside `size` first.
  if (std::string err = check_elf_image(b, size); !err.empty()) {
    return fail(KHRT_E_INVALID, "khrt_module_load_data: " + err);
  }
  if (int rc = ensure_device()) return rc;
  // The HIP runtime may read the image after hipModuleLoadData returns
  // (code objects are loaded lazily), so the caller's buffer must outlive
  // the module. Keep a private copy until khrt_module_unload instead, so a
  // caller may free its image right after this call.
  std::unique_ptr<unsigned char[], void (*)(void *)> copy(
      static_cast<unsigned char *>(std::aligned_alloc(4096, (size + 4095) / 4096 * 4096)), std::free);
  if (!copy) return fail(KHRT_E_INVALID, "khrt_module_load_data: out of host memory");
  std::memcpy(copy.get(), image, size);
  hipModule_t m = nullptr;
  const hipError_t e = hipModuleLoadData(&m, copy.get());
  if (e != hipSuccess) return fail_hip(e, "hipModuleLoadData");
  {
    std::lock_guard<std::mutex> lock(g_mu);
    g_images.emplace(static_cast<void *>(m), std::move(copy));
  }
  *module = m;
  return 0;
}

int khrt_elf_image_size(const void *image, size_t *size) {
  if (image == nullptr || size == nullptr) return fail(KHRT_E_INVALID, "khrt_elf_image_size: null argument");
  *size = 0;
  const unsigned char *b = static_cast<const unsigned char *>(image);
  if (!(b[0] == 0x7f && b[1] == 'E' && b[2] == 'L' && b[3] == 'F')) {
    return fail(KHRT_E_INVALID, "khrt_elf_image_size: image is not an ELF code object");
  }
  auto rd16 = [&](size_t off) { uint16_t v; std::memcpy(&v, b + off, 2); return v; };
  auto rd32 = [&](size_t off) { uint32_t v; std::memcpy(&v, b + off, 4); return v; };
  auto rd64 = [&](size_t off) { uint64_t v; std::memcpy(&v, b + off, 8); return v; };
  if (b[4] != 2 || b[5] != 1 || rd16(18) != 0xE0) {
    return fail(KHRT_E_INVALID, "khrt_elf_image_size: image is not a 64-bit little-endian AMDGPU code object");
  }
  // No code object of this runtime comes near this; larger extents come
  // from headers that are not a code object's.
  constexpr uint64_t kMax = uint64_t(1) << 30;
  const uint64_t phoff = rd64(32), shoff = rd64(40);
  const uint16_t phentsize = rd16(54), phnum = rd16(56), shentsize = rd16(58), shnum = rd16(60);
  if ((phnum > 0 && (phentsize < 56 || phoff > kMax)) || (shnum > 0 && (shentsize < 64 || shoff > kMax))) {
    return fail(KHRT_E_INVALID, "khrt_elf_image_size: malformed header tables");
  }
  uint64_t end = 64;
  auto extend = [&](uint64_t off, uint64_t len) {
    if (off > kMax || len > kMax) return false;
    end = std::max(end, off + len);
    return true;
  };
  bool ok = extend(phoff, uint64_t(phentsize) * phnum) && extend(shoff, uint64_t(shentsize) * shnum);
  for (uint16_t i = 0; ok && i < phnum; ++i) {
    const size_t p = phoff + size_t(i) * phentsize;
    ok = extend(rd64(p + 8), rd64(p + 32));
  }
  for (uint16_t i = 0; ok && i < shnum; ++i) {
    const size_t sh = shoff + size_t(i) * shentsize;
    const uint32_t type = rd32(sh + 4);
    if (type != 8 /* SHT_NOBITS */ && type != 0) ok = extend(rd64(sh + 24), rd64(sh + 32));
  }
  if (!ok || end > kMax) return fail(KHRT_E_INVALID, "khrt_elf_image_size: extent beyond 1 GiB");
  *size = static_cast<size_t>(end);
  return 0;
}

int khrt_module_get_function(void **function, void *module, const char *name) {
  if (function == nullptr || module == nullptr || name == nullptr) {
    return fail(KHRT_E_INVALID, "khrt_module_get_function: null argument");
  }
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, static_cast<hipModule_t>(module), name);
  if (e != hipSuccess) {
    return fail(static_cast<int>(e), std::string("hipModuleGetFunction(\"") + name + "\"): " + hipGetErrorString(e));
  }
  *function = f;
  return 0;
}

int khrt_module_unload(void *module) {
  if (module == nullptr) return fail(KHRT_E_INVALID, "khrt_module_unload: null module");
  const hipError_t e = hipModuleUnload(static_cast<hipModule_t>(module));
  if (e != hipSuccess) return fail_hip(e, "hipModuleUnload");
  std::lock_guard<std::mutex> lock(g_mu);
  g_images.erase(module);  // the private image copy goes with the module
  clear_occupancy_cache();
  return 0;
}

int khrt_launch_raw(void *function, khrt_dim3 grid, khrt_dim3 block, size_t shared_bytes, void *stream,
                    void **params) {
  if (function == nullptr) return fail(KHRT_E_INVALID, "khrt_launch_raw: null function");
  const hipError_t e =
      hipModuleLaunchKernel(static_cast<hipFunction_t>(function), grid.x, grid.y, grid.z, block.x, block.y,
                            block.z, static_cast<unsigned>(shared_bytes), static_cast<hipStream_t>(stream), params,
                            nullptr);
  return e == hipSuccess ? 0 : fail_hip(e, "hipModuleLaunchKernel");
}

int khrt_kernel_launch(void *function, khrt_dim3 grid, khrt_dim3 block, size_t shared_bytes, void *stream,
                       void **params, size_t param_count) {
  return verified_launch(function, grid, block, shared_bytes, stream, params, param_count);
}

int khrt_stream_create(void **stream) {
  if (stream == nullptr) return fail(KHRT_E_INVALID, "khrt_stream_create: null output");
  if (int rc = ensure_device()) return rc;
  hipStream_t s = nullptr;
  const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) return fail_hip(e, "hipStreamCreateWithFlags");
  *stream = s;
  return 0;
}

int khrt_stream_destroy(void *stream) {
  if (stream == nullptr) return 0;
  const hipError_t e = hipStreamDestroy(static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : fail_hip(e, "hipStreamDestroy");
}

int khrt_stream_synchronize(void *stream) {
  const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : fail_hip(e, "hipStreamSynchronize");
}

int khrt_event_create(void **event) {
  if (event == nullptr) return fail(KHRT_E_INVALID, "khrt_event_create: null output");
  if (int rc = ensure_device()) return rc;
  hipEvent_t ev = nullptr;
  const hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) return fail_hip(e, "hipEventCreate");
  *event = ev;
  return 0;
}

int khrt_event_record(void *event, void *stream) {
  if (event == nullptr) return fail(KHRT_E_INVALID, "khrt_event_record: null event");
  const hipError_t e = hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : fail_hip(e, "hipEventRecord");
}

int khrt_event_synchronize(void *event) {
  if (event == nullptr) return fail(KHRT_E_INVALID, "khrt_event_synchronize: null event");
  const hipError_t e = hipEventSynchronize(static_cast<hipEvent_t>(event));
  return e == hipSuccess ? 0 : fail_hip(e, "hipEventSynchronize");
}

int khrt_event_elapsed_ms(float *ms, void *start, void *end) {
  if (ms == nullptr || start == nullptr || end == nullptr) {
    return fail(KHRT_E_INVALID, "khrt_event_elapsed_ms: null argument");
  }
  const hipError_t e = hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end));
  return e == hipSuccess ? 0 : fail_hip(e, "hipEventElapsedTime");
}

int khrt_event_destroy(void *event) {
  if (event == nullptr) return 0;
  const hipError_t e = hipEventDestroy(static_cast<hipEvent_t>(event));
  return e == hipSuccess ? 0 : fail_hip(e, "hipEventDestroy");
}

size_t khrt_memref_slot_count(int rank) { return rank < 0 ? 0 : static_cast<size_t>(2 * rank + 3); }

int khrt_pack_memref(uint64_t *slots, size_t cap, const void *dev_ptr, int rank, const int64_t *shape) {
  if (slots == nullptr || rank < 0 || (rank > 0 && shape == nullptr)) {
    return fail(KHRT_E_INVALID, "khrt_pack_memref: null slots/shape or negative rank");
  }
  if (cap < khrt_memref_slot_count(rank)) {
    return fail(KHRT_E_INVALID, "khrt_pack_memref: capacity " + std::to_string(cap) + " < " +
                                    std::to_string(khrt_memref_slot_count(rank)) + " slots");
  }
  LaunchArgs a;
  a.add_memref(dev_ptr, std::vector<int64_t>(shape, shape + rank));
  std::memcpy(slots, a.slots().data(), a.slots().size() * sizeof(uint64_t));
  return 0;
}

int khrt_pack_scalar(uint64_t *slot, const void *value, size_t byte_size) {
  if (slot == nullptr) return fail(KHRT_E_INVALID, "khrt_pack_scalar: null slot");
  if (byte_size > 8) return fail(KHRT_E_INVALID, "khrt_pack_scalar: scalars are at most 8 bytes");
  LaunchArgs a;
  a.add_scalar_bytes(value, byte_size);
  *slot = a.slots()[0];
  return 0;
}

}  // extern "C"
