// Roofline microbenchmarks for gfx950: the measured ceilings the kernels'
// fractions are quoted against. Replaces the reference's roofline_triad and
// roofline_fma comparators (bench/refs/roofline.hip:22-53, driven by
// bench/harness/roofline.cpp:60-130) with MI355X-shaped ones:
//
//   roofline_triad  c = a + b over >= 3 GiB (beyond the 256 MB Infinity
//                   Cache): 12 B per element.
//   roofline_copy   dst = src: a kernel of exactly known traffic, used to
//                   calibrate the FETCH_SIZE / WRITE_SIZE counters.
//   roofline_mfma   back-to-back independent v_mfma_f32_32x32x2f32 chains
//   roofline_mfma16 the same with v_mfma_f32_16x16x4f32
//                   per wave (4096 FLOP each), no memory traffic in the
//                   loop: the attainable fp32 matrix rate.
//
// The streaming pair uses the fastest pattern a sweep over unroll depth,
// cache hints and grid size found on MI355X: four nontemporal dwordx4 loads
// in flight per thread before the stores, 32 workgroups per CU.
#include "kh_device.h"

typedef float v16f __attribute__((ext_vector_type(16)));

namespace {
constexpr int kU = 4;
}

extern "C" __global__ void __launch_bounds__(256)
roofline_triad(KH_MEMREF1(const float, a), KH_MEMREF1(const float, b), KH_MEMREF1(float, c)) {
  const float *__restrict__ A = KH_PTR(a);
  const float *__restrict__ B = KH_PTR(b);
  float *__restrict__ C = KH_PTR(c);
  const int64_t n4 = c_n0 >> 2;
  const int64_t bd = blockDim.x;
  const int64_t step = bd * gridDim.x * kU;
  for (int64_t i = (int64_t)blockIdx.x * bd * kU + threadIdx.x; i + (kU - 1) * bd < n4; i += step) {
    float4 x[kU], y[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      x[u] = kh::load_nt(A + 4 * (i + u * bd));
      y[u] = kh::load_nt(B + 4 * (i + u * bd));
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
      kh::store_nt(C + 4 * (i + u * bd), make_float4(x[u].x + y[u].x, x[u].y + y[u].y, x[u].z + y[u].z, x[u].w + y[u].w));
  }
  // Vectors past the last full unrolled step.
  const int64_t done = (n4 / (bd * kU)) * (bd * kU);
  for (int64_t i = done + (int64_t)blockIdx.x * bd + threadIdx.x; i < n4; i += bd * gridDim.x) {
    const float4 x = kh::load_nt(A + 4 * i), y = kh::load_nt(B + 4 * i);
    kh::store_nt(C + 4 * i, make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w));
  }
}

extern "C" __global__ void __launch_bounds__(256)
roofline_copy(KH_MEMREF1(const float, src), KH_MEMREF1(float, dst)) {
  const float *__restrict__ S = KH_PTR(src);
  float *__restrict__ T = KH_PTR(dst);
  const int64_t n4 = dst_n0 >> 2;
  const int64_t bd = blockDim.x;
  const int64_t step = bd * gridDim.x * kU;
  for (int64_t i = (int64_t)blockIdx.x * bd * kU + threadIdx.x; i + (kU - 1) * bd < n4; i += step) {
    float4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = kh::load_nt(S + 4 * (i + u * bd));
#pragma unroll
    for (int u = 0; u < kU; ++u) kh::store_nt(T + 4 * (i + u * bd), v[u]);
  }
  // Vectors past the last full unrolled step.
  const int64_t done = (n4 / (bd * kU)) * (bd * kU);
  for (int64_t i = done + (int64_t)blockIdx.x * bd + threadIdx.x; i < n4; i += bd * gridDim.x)
    kh::store_nt(T + 4 * i, kh::load_nt(S + 4 * i));
}

// out[n0 >= blocks*threads]: one value per thread keeps the chains live.
// Each wave runs `iters` rounds of 8 independent MFMAs.
extern "C" __global__ void __launch_bounds__(256)
roofline_mfma(KH_MEMREF1(float, out), int64_t iters) {
  const int lane = kh::lane_id();
  const float a = 1.0f + 1e-7f * (float)lane, b = 1.0f - 1e-7f * (float)lane;
  v16f acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = v16f{};
  for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid < out_n0) KH_PTR(out)[gid] = s;
}

// The same with v_mfma_f32_16x16x4f32 (the same rate per CU, a quarter of the
// work per instruction): 16 independent chains per wave.
typedef float v4f __attribute__((ext_vector_type(4)));
extern "C" __global__ void __launch_bounds__(256)
roofline_mfma16(KH_MEMREF1(float, out), int64_t iters) {
  const int lane = kh::lane_id();
  const float a = 1.0f + 1e-7f * (float)lane, b = 1.0f - 1e-7f * (float)lane;
  v4f acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = v4f{};
  for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) s += acc[j][r];
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid < out_n0) KH_PTR(out)[gid] = s;
}
