// fused_gelu for gfx950: out = gelu_tanh(1.5 x + 0.5), fp32, HBM-bound
// (read x, write out: 8 B/element).
//
// Symbol and memref arguments follow the reference template
// (lib/dsl/kernels/fused_gelu.cpp:73-160): x, tmp, out, rank-1 [n], 15
// parameters. After the reference's fuse pass the producer's store to `tmp`
// is gone (lib/passes/fusion.cpp:331-333), so `tmp` is a dead argument here
// too: it is never read or written.
//
// Arithmetic (fused_gelu.cpp:113-119, 137-156):
//   t = 1.5 x + 0.5
//   z = 0.7978845608 (t + 0.044715 t^3)
//   out = 0.5 t (1 + tanh z)
// tanh is evaluated from the identity 1 + tanh z = 2 - 2 / (1 + e^{2z}),
// with e^{2z} = 2^{2 z log2 e} on v_exp_f32 and the division as a multiply
// by v_rcp_f32 (the hardware's approximate reciprocal, 1 ulp); e^{2z}
// overflowing to +inf gives exactly 2 (rcp(inf) = 0), underflowing to 0
// gives exactly 0, so the formula is finite for every finite input. The
// absolute error of out is a few fp32 ulps of |t|, far inside the 1e-4
// fp64-reference tolerance (e2e_fused_gelu_test.cpp:63).
#include <type_traits>

#include "kh_device.h"
#include "kh_tiles.h"

#define KH_UNROLL KH_EW_UNROLL

namespace {

__device__ __forceinline__ float gelu_affine(float x) {
  const float t = fmaf(1.5f, x, 0.5f);
  const float t3 = t * t * t;
  const float z = 0.7978845608f * fmaf(0.044715f, t3, t);
  const float e = kh::exp2_hw(z * (2.0f * kh::kLog2e));
  const float one_plus_tanh = 2.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + e);
  return 0.5f * t * one_plus_tanh;
}

__device__ __forceinline__ float4 gelu4(float4 v) {
  float4 r;
  r.x = gelu_affine(v.x);
  r.y = gelu_affine(v.y);
  r.z = gelu_affine(v.z);
  r.w = gelu_affine(v.w);
  return r;
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256)
fused_gelu(KH_MEMREF1(const float, x), KH_MEMREF1(float, tmp), KH_MEMREF1(float, out)) {
  (void)tmp_alloc;
  (void)tmp_base;
  const uint32_t gw = kh::group_size_word(), blocks = kh::grid_blocks_x();
  KH_ARGS_READY(x_base, x_off, out_base, out_off, out_n0, gw, blocks);
  const float *__restrict__ X = KH_PTR(x);
  float *__restrict__ O = KH_PTR(out);
  const int64_t n = out_n0;
  const int64_t bd = kh::threads_x_of(gw);
  const int64_t nb = blocks;
  const int64_t tid = threadIdx.x;
  const int64_t gid = (int64_t)blockIdx.x * bd + tid;

  if (kh::aligned16(X) && kh::aligned16(O)) {
    // Streamed once, nontemporal, KH_UNROLL float4 per thread: the
    // launcher's grid covers n in one step of the (scalar) loop; smaller
    // grids take more steps. Each step moves through buffer resources over
    // exactly the workgroup's float4s inside n, so the ragged end needs no
    // branches. In a launch that fits one round, the first step's loads go
    // out in two halves, the second once the first has landed, and its
    // stores once all have (kh::kFirstBurst).
    const int64_t n4 = n >> 2;
    const int64_t per_step = bd * KH_UNROLL;
    auto step = [&](auto split_tag, int64_t b0) __attribute__((always_inline)) {
      constexpr bool kSplit = decltype(split_tag)::value;
      const uint32_t bytes = (uint32_t)((n4 - b0 < per_step ? n4 - b0 : per_step) * 16);
      const __amdgpu_buffer_rsrc_t rx = kh::span_rsrc(X + 4 * b0, bytes);
      const __amdgpu_buffer_rsrc_t ro = kh::span_rsrc(O + 4 * b0, bytes);
      float4 v[KH_UNROLL];
#pragma unroll
      for (int u = 0; u < KH_UNROLL; ++u) {
        v[u] = kh::buf_load4_nt(rx, (uint32_t)(tid + u * bd) * 16u);
        if (kSplit && u + 1 == kh::kFirstBurst) kh::vm_wait<0>();
      }
      if (kSplit) kh::vm_wait<0>();
#pragma unroll
      for (int u = 0; u < KH_UNROLL; ++u) kh::buf_store4_nt(ro, (uint32_t)(tid + u * bd) * 16u, gelu4(v[u]));
    };
    int64_t b0 = (int64_t)blockIdx.x * per_step;
    if (b0 < n4) {
      if (kh::split_first_burst(bd * nb))
        step(std::true_type{}, b0);
      else
        step(std::false_type{}, b0);
    }
    for (b0 += nb * per_step; b0 < n4; b0 += nb * per_step) step(std::false_type{}, b0);
    const int64_t t = (n4 << 2) + gid;
    if (t < n) O[t] = gelu_affine(X[t]);
  } else {
    for (int64_t i = gid; i < n; i += bd * nb) O[i] = gelu_affine(X[i]);
  }
}
