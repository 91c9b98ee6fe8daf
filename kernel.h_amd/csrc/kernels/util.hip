// Runtime utility kernels (not templates): a float fill used by the host
// runtime where a memset would not be safe under stream capture.
#include "kh_device.h"

extern "C" __global__ void __launch_bounds__(256)
kh_fill_f32(KH_MEMREF1(float, dst), float value) {
  float *__restrict__ D = KH_PTR(dst);
  const int64_t n = dst_n0;
  const int64_t stride = (int64_t)blockDim.x * gridDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) D[i] = value;
}
