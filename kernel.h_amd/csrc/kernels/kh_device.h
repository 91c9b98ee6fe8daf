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

// Launch geometry from the implicit kernel arguments, one 32-bit scalar load
// each (code object v5: hidden_block_count_x, a u32 at byte 0, and
// hidden_group_size_x, a u16 at byte 12; HIP launches whole workgroups, so
// the group size is the block size). blockDim.x can compile into a 16-bit
// vector load (gfx9 has no 16-bit scalar load) that the prologue must wait
// for: another serial round trip to kernel-argument memory, about 0.5-1 us
// at the start of every launch, before its first data load can issue.
__device__ __forceinline__ uint32_t implicit_arg_u32(int index) {
  const uint32_t __attribute__((address_space(4))) *p =
      (const uint32_t __attribute__((address_space(4))) *)__builtin_amdgcn_implicitarg_ptr();
  return p[index];
}
// Raw words: the block counts, the word holding the workgroup's x and y
// sizes (16 bits each: threads_x_of, threads_y_of) and the one whose low 16
// bits are its z size (threads_z_of).
__device__ __forceinline__ uint32_t grid_blocks_x() { return implicit_arg_u32(0); }
__device__ __forceinline__ uint32_t grid_blocks_y() { return implicit_arg_u32(1); }
__device__ __forceinline__ uint32_t grid_blocks_z() { return implicit_arg_u32(2); }
__device__ __forceinline__ uint32_t group_size_word() { return implicit_arg_u32(3); }
__device__ __forceinline__ uint32_t group_size_z_word() { return implicit_arg_u32(4); }
__device__ __forceinline__ uint32_t threads_x_of(uint32_t word) { return word & 0xffffu; }
__device__ __forceinline__ uint32_t threads_y_of(uint32_t word) { return word >> 16; }
__device__ __forceinline__ uint32_t threads_z_of(uint32_t word) { return word & 0xffffu; }
__device__ __forceinline__ uint32_t block_threads_x() { return threads_x_of(group_size_word()); }

}  // namespace kh

// KH_ARGS_READY(v...): issues the scalar loads behind the given values here,
// all in one round, and waits for them once. Pass values exactly as loaded
// (descriptor fields, raw implicit-argument words): arithmetic on a loaded
// value before this point makes the compiler wait for that load first and
// issue the rest after it. The values keep their identity (pointers keep
// their global address space): the empty asm only reads them. Left alone,
// the compiler sinks each kernel-argument load past the branches to where it
// is first used, and every load it sinks behind a wait adds a serial round
// trip to kernel-argument memory (cold at the start of a launch) before the
// first data load can issue.
#define KH_S_OP(v) "s"(v)
#define KH_FE_1(M, a) M(a)
#define KH_FE_2(M, a, ...) M(a), KH_FE_1(M, __VA_ARGS__)
#define KH_FE_3(M, a, ...) M(a), KH_FE_2(M, __VA_ARGS__)
#define KH_FE_4(M, a, ...) M(a), KH_FE_3(M, __VA_ARGS__)
#define KH_FE_5(M, a, ...) M(a), KH_FE_4(M, __VA_ARGS__)
#define KH_FE_6(M, a, ...) M(a), KH_FE_5(M, __VA_ARGS__)
#define KH_FE_7(M, a, ...) M(a), KH_FE_6(M, __VA_ARGS__)
#define KH_FE_8(M, a, ...) M(a), KH_FE_7(M, __VA_ARGS__)
#define KH_FE_9(M, a, ...) M(a), KH_FE_8(M, __VA_ARGS__)
#define KH_FE_10(M, a, ...) M(a), KH_FE_9(M, __VA_ARGS__)
#define KH_FE_11(M, a, ...) M(a), KH_FE_10(M, __VA_ARGS__)
#define KH_FE_12(M, a, ...) M(a), KH_FE_11(M, __VA_ARGS__)
#define KH_FE_13(M, a, ...) M(a), KH_FE_12(M, __VA_ARGS__)
#define KH_FE_14(M, a, ...) M(a), KH_FE_13(M, __VA_ARGS__)
#define KH_FE_15(M, a, ...) M(a), KH_FE_14(M, __VA_ARGS__)
#define KH_FE_16(M, a, ...) M(a), KH_FE_15(M, __VA_ARGS__)
#define KH_FE_17(M, a, ...) M(a), KH_FE_16(M, __VA_ARGS__)
#define KH_FE_18(M, a, ...) M(a), KH_FE_17(M, __VA_ARGS__)
#define KH_FE_19(M, a, ...) M(a), KH_FE_18(M, __VA_ARGS__)
#define KH_FE_20(M, a, ...) M(a), KH_FE_19(M, __VA_ARGS__)
#define KH_FE_PICK(_1, _2, _3, _4, _5, _6, _7, _8, _9, _10, _11, _12, _13, _14, _15, _16, _17, _18, _19, _20, NAME, \
                   ...)                                                                                        \
  NAME
#define KH_FOR_EACH(M, ...)                                                                                    \
  KH_FE_PICK(__VA_ARGS__, KH_FE_20, KH_FE_19, KH_FE_18, KH_FE_17, KH_FE_16, KH_FE_15, KH_FE_14, KH_FE_13,      \
             KH_FE_12, KH_FE_11, KH_FE_10, KH_FE_9, KH_FE_8, KH_FE_7, KH_FE_6, KH_FE_5, KH_FE_4, KH_FE_3,       \
             KH_FE_2, KH_FE_1)(M, __VA_ARGS__)
#define KH_ARGS_READY(...) asm volatile("" ::KH_FOR_EACH(KH_S_OP, __VA_ARGS__))

namespace kh {

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

// Buffer access to a span of `bytes` bytes from p (32-bit data format): the
// hardware range check makes loads past the end read 0 and drops stores past
// it, so ragged edges need no per-lane branches and the loads a path issues
// are exactly the ones written (a branch around a load makes the compiler
// wait for every load in flight where the paths join).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
constexpr int kBufNt = 2;  // buffer cache-policy operand: nontemporal (gfx940+ nt bit)
__device__ __forceinline__ float4 buf_load4_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4_t u = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kBufNt);
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
}
__device__ __forceinline__ void buf_store4_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 f) {
  const u32x4_t u = {__float_as_uint(f.x), __float_as_uint(f.y), __float_as_uint(f.z), __float_as_uint(f.w)};
  __builtin_amdgcn_raw_buffer_store_b128(u, r, off, 0, kBufNt);
}

// Waits until at most N vector-memory operations of this wave are in flight
// (gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at
// [15:14]; expcnt and lgkmcnt left at "no wait").
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 63, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Streaming kernels at 33.5 MB (4096 waves of four 1 KiB loads each, one
// launch, MI355X): issuing each wave's loads in two halves, the second once
// the first has landed, ran 6.05-6.13 us against 6.9-7.1 us with all four
// in flight at once and 6.7-6.9 us one at a time (copy and softmax alike,
// same bits). The smaller first burst over the whole chip is what helps, so
// the split applies to the first step of launches that fit one round of the
// chip (256 CUs x 2048 resident threads): in longer launches every wave
// keeping all its loads in flight moves more bytes, and in a later step of a
// loop the wait would also hold for the previous step's stores (vector
// memory operations retire in issue order).
constexpr int kFirstBurst = 2;
constexpr int64_t kFirstBurstMaxThreads = 256 * 2048;
__device__ __forceinline__ bool split_first_burst(int64_t launch_threads) {
  return launch_threads <= kFirstBurstMaxThreads;
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
