// Shared device-side helpers for the gfx950 (CDNA4, wave64) kernel.h
// templates: memref-descriptor parameter lists and wavefront reductions.
//
// Kernel ABI. Every buffer argument arrives as the expanded MLIR memref
// descriptor the reference emitter produces (lib/compiler/emitter.cpp:
// 713-727; lib/runtime/descriptor_packing.cpp:3-39): 2N+3 eight-byte kernel
// parameters {allocated ptr, aligned ptr, offset, sizes[N], strides[N]}.
// Element (i0..iN-1) lives at aligned + offset + sum(ik * stride_k). The
// launcher always packs contiguous row-major descriptors with offset 0, and
// the kernels honour the offset and the outer strides.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define KH_MEMREF1(T, name) \
  T *__restrict__ name##_alloc, T *__restrict__ name##_base, int64_t name##_off, int64_t name##_n0, int64_t name##_s0

#define KH_MEMREF2(T, name)                                                                 \
  T *__restrict__ name##_alloc, T *__restrict__ name##_base, int64_t name##_off, int64_t name##_n0, \
      int64_t name##_n1, int64_t name##_s0, int64_t name##_s1

#define KH_MEMREF4(T, name)                                                                 \
  T *__restrict__ name##_alloc, T *__restrict__ name##_base, int64_t name##_off, int64_t name##_n0, \
      int64_t name##_n1, int64_t name##_n2, int64_t name##_n3, int64_t name##_s0, int64_t name##_s1, \
      int64_t name##_s2, int64_t name##_s3

// Element pointer of a descriptor (aligned pointer + offset).
#define KH_PTR(name) (name##_base + name##_off)

namespace kh {

constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// DPP row_ror:n (rotate right by n within each 16-lane row), gfx9 encoding
// 0x120 + n. All rows and banks enabled; rotation never leaves the row.
template <int N>
__device__ __forceinline__ float ror(float v) {
  static_assert(N >= 1 && N <= 15, "row_ror range");
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x120 + N, 0xf, 0xf, false));
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Wavefront all-reduce: a rotate-and-combine butterfly inside each 16-lane
// row (every lane ends with its row's total), then the four row totals are
// read into scalar registers and combined. The result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
  v += ror<8>(v);
  v += ror<4>(v);
  v += ror<2>(v);
  v += ror<1>(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, ror<8>(v));
  v = fmaxf(v, ror<4>(v));
  v = fmaxf(v, ror<2>(v));
  v = fmaxf(v, ror<1>(v));
  return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}

// dwordx4 loads/stores with the nontemporal hint: streamed data that is
// touched once should not displace reusable lines in L2 / the MALL. On
// MI355X this lifts streaming kernels from ~5.4 to ~5.9-6.1 TB/s.
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 load_nt(const float *p) {
  const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void store_nt(float *p, float4 f) {
  const v4f v = {f.x, f.y, f.z, f.w};
  __builtin_nontemporal_store(v, reinterpret_cast<v4f *>(p));
}

// 2^x on the hardware transcendental unit (v_exp_f32).
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

// Workgroup barrier that orders LDS accesses only. __syncthreads() is a
// workgroup-scope release/acquire fence on all memory, which makes every
// wave wait for its outstanding global loads and stores at the barrier;
// kernels whose waves share data through LDS alone use this instead, so
// prefetches and stores stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace kh
