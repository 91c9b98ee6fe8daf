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
// The streaming pair uses the fastest pattern found on MI355X: four
// nontemporal dwordx4 accesses per thread and operand, the loads issued in two
// halves (the second once the first has landed), then the stores; bench.py
// runs it at one step per workgroup and at 32 grid-strided workgroups per CU.
#include "kh_device.h"

typedef float v16f __attribute__((ext_vector_type(16)));

namespace {
constexpr int kU = 4;
}

// One unrolled step per workgroup: bd x kU float4s through buffer spans over
// exactly the step's elements (the ragged end needs no branches), nontemporal,
// the first step's loads in two halves when the launch fits one round
// (kh::kFirstBurst), as in the product streaming kernels; smaller grids loop
// over steps.
namespace {
// One step of the stream over the float4s [s0, s0 + bd kU) within n4, for
// N = 1 (copy) or 2 (triad) source operands.
template <int N, bool SPLIT>
__device__ __forceinline__ void stream_step(const float *__restrict__ A, const float *__restrict__ B,
                                            float *__restrict__ C, int64_t n4, int64_t s0, int64_t per,
                                            uint32_t bd, uint32_t tid) {
  const uint32_t bytes = (uint32_t)((n4 - s0 < per ? n4 - s0 : per) * 16);
  const __amdgpu_buffer_rsrc_t ra = kh::span_rsrc(A + 4 * s0, bytes), rc = kh::span_rsrc(C + 4 * s0, bytes);
  const __amdgpu_buffer_rsrc_t rb = kh::span_rsrc(N == 2 ? B + 4 * s0 : A, N == 2 ? bytes : 0);
  float4 x[kU], y[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    x[u] = kh::buf_load4_nt(ra, (tid + u * bd) * 16u);
    if (N == 2) y[u] = kh::buf_load4_nt(rb, (tid + u * bd) * 16u);
    if (SPLIT && u + 1 == kU / 2) kh::vm_wait<0>();
  }
  if (SPLIT) kh::vm_wait<0>();
#pragma unroll
  for (int u = 0; u < kU; ++u)
    kh::buf_store4_nt(rc, (tid + u * bd) * 16u,
                      N == 2 ? make_float4(x[u].x + y[u].x, x[u].y + y[u].y, x[u].z + y[u].z, x[u].w + y[u].w)
                             : x[u]);
}

template <int N>
__device__ __forceinline__ void stream(const float *__restrict__ A, const float *__restrict__ B,
                                       float *__restrict__ C, int64_t n, uint32_t gw, uint32_t nb) {
  const int64_t n4 = n >> 2, bd = kh::threads_x_of(gw), per = bd * kU;
  const uint32_t tid = threadIdx.x;
  int64_t s0 = (int64_t)blockIdx.x * per;
  if (s0 < n4) {
    if (kh::split_first_burst(bd * (int64_t)nb))
      stream_step<N, true>(A, B, C, n4, s0, per, (uint32_t)bd, tid);
    else
      stream_step<N, false>(A, B, C, n4, s0, per, (uint32_t)bd, tid);
  }
  for (s0 += (int64_t)nb * per; s0 < n4; s0 += (int64_t)nb * per)
    stream_step<N, false>(A, B, C, n4, s0, per, (uint32_t)bd, tid);
}
}  // namespace

// One unrolled step per workgroup: bd x kU float4s through buffer spans over
// exactly the step's elements (the ragged end needs no branches), nontemporal.
// In a launch that fits one round the first step's loads go out in two
// halves and its stores once all have landed (kh::kFirstBurst), as in the
// product streaming kernels; smaller grids loop over steps.
extern "C" __global__ void __launch_bounds__(256)
roofline_triad(KH_MEMREF1(const float, a), KH_MEMREF1(const float, b), KH_MEMREF1(float, c)) {
  const uint32_t gw = kh::group_size_word(), nb = kh::grid_blocks_x();
  KH_ARGS_READY(a_base, a_off, b_base, b_off, c_base, c_off, c_n0, gw, nb);
  stream<2>(KH_PTR(a), KH_PTR(b), KH_PTR(c), c_n0, gw, nb);
}

extern "C" __global__ void __launch_bounds__(256)
roofline_copy(KH_MEMREF1(const float, src), KH_MEMREF1(float, dst)) {
  const uint32_t gw = kh::group_size_word(), nb = kh::grid_blocks_x();
  KH_ARGS_READY(src_base, src_off, dst_base, dst_off, dst_n0, gw, nb);
  stream<1>(KH_PTR(src), nullptr, KH_PTR(dst), dst_n0, gw, nb);
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
