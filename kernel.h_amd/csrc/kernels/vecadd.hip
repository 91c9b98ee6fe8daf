// vecadd for gfx950: c[i] = a[i] + b[i], fp32, HBM-bound (12 B/element).
//
// Same symbol and memref arguments as the reference template
// (lib/dsl/kernels/vecadd.cpp:44-89): three rank-1 [n] f32 descriptors,
// 15 kernel parameters. The reference body is a scalar grid-stride loop
// (vecadd.cpp:71-88); here each thread moves KH_UNROLL dwordx4 vectors per
// grid-stride step, all loads issued before the adds, so every wave keeps
// several 1 KiB requests in flight. The grid-stride form keeps the kernel
// correct under any launch geometry, including the reference's
// ceil(n/256) x 256 (e2e_vecadd_test.cpp:90-92).
//
// Result: one IEEE fp32 add per element, bit-identical to the fp64 sum
// rounded to fp32 for every finite input.
#include "kh_device.h"

#ifndef KH_UNROLL
#define KH_UNROLL 4
#endif

extern "C" __global__ void __launch_bounds__(256)
vecadd(KH_MEMREF1(const float, a), KH_MEMREF1(const float, b), KH_MEMREF1(float, c)) {
  const float *__restrict__ A = KH_PTR(a);
  const float *__restrict__ B = KH_PTR(b);
  float *__restrict__ C = KH_PTR(c);
  const int64_t n = c_n0;
  const int64_t tid = threadIdx.x;
  const int64_t nthreads = (int64_t)blockDim.x * gridDim.x;

  if (kh::aligned16(A) && kh::aligned16(B) && kh::aligned16(C)) {
    const int64_t n4 = n >> 2;
    const float4 *__restrict__ A4 = reinterpret_cast<const float4 *>(A);
    const float4 *__restrict__ B4 = reinterpret_cast<const float4 *>(B);
    float4 *__restrict__ C4 = reinterpret_cast<float4 *>(C);
    const int64_t step = nthreads * KH_UNROLL;
    int64_t i = (int64_t)blockIdx.x * blockDim.x * KH_UNROLL + tid;
    for (; i + (KH_UNROLL - 1) * (int64_t)blockDim.x < n4; i += step) {
      float4 va[KH_UNROLL], vb[KH_UNROLL];
#pragma unroll
      for (int u = 0; u < KH_UNROLL; ++u) {
        va[u] = A4[i + u * (int64_t)blockDim.x];
        vb[u] = B4[i + u * (int64_t)blockDim.x];
      }
#pragma unroll
      for (int u = 0; u < KH_UNROLL; ++u) {
        float4 r;
        r.x = va[u].x + vb[u].x;
        r.y = va[u].y + vb[u].y;
        r.z = va[u].z + vb[u].z;
        r.w = va[u].w + vb[u].w;
        C4[i + u * (int64_t)blockDim.x] = r;
      }
    }
    // Remainder of the vector range: at most KH_UNROLL-1 partial groups.
    for (int u = 0; u < KH_UNROLL; ++u) {
      const int64_t j = i + u * (int64_t)blockDim.x;
      if (j < n4) {
        const float4 x = A4[j], y = B4[j];
        float4 r;
        r.x = x.x + y.x;
        r.y = x.y + y.y;
        r.z = x.z + y.z;
        r.w = x.w + y.w;
        C4[j] = r;
      }
    }
    // Scalar tail (n % 4 elements), one thread each.
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + tid;
    const int64_t t = (n4 << 2) + gid;
    if (t < n) C[t] = A[t] + B[t];
  } else {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + tid; i < n; i += nthreads) C[i] = A[i] + B[i];
  }
}
