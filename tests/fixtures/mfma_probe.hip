// Test-only code object (never part of the product registry): exposes the
// fp32 MFMA builtins one instruction at a time so a GPU test can check the
// operand/result lane layouts the gemm and attention kernels rely on.
// Each lane passes its own A and B operand values; the kernel writes the
// accumulator registers unchanged (out[lane * R + r]). One wavefront.
#include "kh_device.h"

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

extern "C" __global__ void __launch_bounds__(64)
probe_mfma_32x32x2(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ out) {
  const int l = threadIdx.x;
  v16f acc = {};
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[l], b[l], acc, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 16; ++r) out[l * 16 + r] = acc[r];
}

extern "C" __global__ void __launch_bounds__(64)
probe_mfma_16x16x4(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ out) {
  const int l = threadIdx.x;
  v4f acc = {};
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[l], b[l], acc, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 4; ++r) out[l * 4 + r] = acc[r];
}
