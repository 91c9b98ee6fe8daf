// vecadd for gfx950: c[i] = a[i] + b[i], fp32, HBM-bound (12 B/element).
//
// Same symbol and memref arguments as the reference template
// (lib/dsl/kernels/vecadd.cpp:44-89): three rank-1 [n] f32 descriptors,
// 15 kernel parameters. The reference body is a scalar grid-stride loop
// (vecadd.cpp:71-88); here each thread moves KH_EW_UNROLL dwordx4 vectors
// per grid-stride step with nontemporal hints, all loads issued before the
// adds, so every wave keeps several 1 KiB requests in flight and the
// streamed data does not displace reusable cache lines (kernel arguments in
// one round of scalar loads, buffer spans, first-burst split: the streaming
// pattern of kh_device.h). The grid-stride form
// keeps the kernel correct under any launch geometry, including the
// reference's ceil(n/256) x 256 (e2e_vecadd_test.cpp:90-92).
//
// Result: one IEEE fp32 add per element, bit-identical to the fp64 sum
// rounded to fp32 for every finite input.
#include "kh_device.h"
#include "kh_tiles.h"

namespace {
constexpr int kU = KH_EW_UNROLL;

__device__ __forceinline__ float4 add4(float4 x, float4 y) {
  return make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
}
// One unrolled step over the float4s [s0, s0 + bd kU) within n4, through
// buffer spans over exactly the step's elements (the ragged end needs no
// branches). SPLIT (the first step of a launch that fits one round): the
// loads go out in two halves and the stores once all have landed
// (kh::kFirstBurst).
template <bool SPLIT>
__device__ __forceinline__ void add_step(const float *__restrict__ A, const float *__restrict__ B,
                                         float *__restrict__ C, int64_t n4, int64_t s0, int64_t per, uint32_t bd,
                                         uint32_t tid) {
  const uint32_t bytes = (uint32_t)((n4 - s0 < per ? n4 - s0 : per) * 16);
  const __amdgpu_buffer_rsrc_t ra = kh::span_rsrc(A + 4 * s0, bytes), rb = kh::span_rsrc(B + 4 * s0, bytes),
                               rc = kh::span_rsrc(C + 4 * s0, bytes);
  float4 va[kU], vb[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    va[u] = kh::buf_load4_nt(ra, (tid + u * bd) * 16u);
    vb[u] = kh::buf_load4_nt(rb, (tid + u * bd) * 16u);
    if (SPLIT && u + 1 == kU / 2) kh::vm_wait<0>();
  }
  if (SPLIT) kh::vm_wait<0>();
#pragma unroll
  for (int u = 0; u < kU; ++u) kh::buf_store4_nt(rc, (tid + u * bd) * 16u, add4(va[u], vb[u]));
}
}  // namespace

extern "C" __global__ void __launch_bounds__(256)
vecadd(KH_MEMREF1(const float, a), KH_MEMREF1(const float, b), KH_MEMREF1(float, c)) {
  const uint32_t gw = kh::group_size_word(), nb = kh::grid_blocks_x();
  KH_ARGS_READY(a_base, a_off, b_base, b_off, c_base, c_off, c_n0, gw, nb);  // one round of scalar loads
  const float *__restrict__ A = KH_PTR(a);
  const float *__restrict__ B = KH_PTR(b);
  float *__restrict__ C = KH_PTR(c);
  const int64_t n = c_n0;
  const int64_t tid = threadIdx.x;
  const int64_t bd = kh::threads_x_of(gw);
  const int64_t nthreads = bd * nb;

  if (kh::aligned16(A) && kh::aligned16(B) && kh::aligned16(C)) {
    const int64_t n4 = n >> 2, per = bd * kU;
    int64_t s0 = (int64_t)blockIdx.x * per;
    if (s0 < n4) {
      if (kh::split_first_burst(nthreads))
        add_step<true>(A, B, C, n4, s0, per, (uint32_t)bd, (uint32_t)tid);
      else
        add_step<false>(A, B, C, n4, s0, per, (uint32_t)bd, (uint32_t)tid);
    }
    for (s0 += nb * per; s0 < n4; s0 += nb * per) add_step<false>(A, B, C, n4, s0, per, (uint32_t)bd, (uint32_t)tid);
    // Scalar tail (n % 4 elements), one thread each.
    const int64_t gid = (int64_t)blockIdx.x * bd + tid;
    const int64_t t = (n4 << 2) + gid;
    if (t < n) C[t] = A[t] + B[t];
  } else {
    for (int64_t i = (int64_t)blockIdx.x * bd + tid; i < n; i += nthreads) C[i] = A[i] + B[i];
  }
}
