// vecadd for gfx950: c[i] = a[i] + b[i], fp32, HBM-bound (12 B/element).
//
// Same symbol and memref arguments as the reference template
// (lib/dsl/kernels/vecadd.cpp:44-89): three rank-1 [n] f32 descriptors,
// 15 kernel parameters. The reference body is a scalar grid-stride loop
// (vecadd.cpp:71-88); here each thread moves KH_EW_UNROLL dwordx4 vectors
// per grid-stride step with nontemporal hints, all loads issued before the
// adds, so every wave keeps several 1 KiB requests in flight and the
// streamed data does not displace reusable cache lines. The grid-stride form
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
}  // namespace

extern "C" __global__ void __launch_bounds__(256)
vecadd(KH_MEMREF1(const float, a), KH_MEMREF1(const float, b), KH_MEMREF1(float, c)) {
  const float *__restrict__ A = KH_PTR(a);
  const float *__restrict__ B = KH_PTR(b);
  float *__restrict__ C = KH_PTR(c);
  const int64_t n = c_n0;
  const int64_t tid = threadIdx.x;
  const int64_t bd = blockDim.x;
  const int64_t nthreads = bd * gridDim.x;

  if (kh::aligned16(A) && kh::aligned16(B) && kh::aligned16(C)) {
    const int64_t n4 = n >> 2;
    const int64_t step = nthreads * kU;
    int64_t i = (int64_t)blockIdx.x * bd * kU + tid;
    for (; i + (kU - 1) * bd < n4; i += step) {
      float4 va[kU], vb[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        va[u] = kh::load_nt(A + 4 * (i + u * bd));
        vb[u] = kh::load_nt(B + 4 * (i + u * bd));
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) kh::store_nt(C + 4 * (i + u * bd), add4(va[u], vb[u]));
    }
    // Remainder of the vector range: at most kU-1 partial groups.
    for (int u = 0; u < kU; ++u) {
      const int64_t j = i + u * bd;
      if (j < n4) kh::store_nt(C + 4 * j, add4(kh::load_nt(A + 4 * j), kh::load_nt(B + 4 * j)));
    }
    // Scalar tail (n % 4 elements), one thread each.
    const int64_t gid = (int64_t)blockIdx.x * bd + tid;
    const int64_t t = (n4 << 2) + gid;
    if (t < n) C[t] = A[t] + B[t];
  } else {
    for (int64_t i = (int64_t)blockIdx.x * bd + tid; i < n; i += nthreads) C[i] = A[i] + B[i];
  }
}
