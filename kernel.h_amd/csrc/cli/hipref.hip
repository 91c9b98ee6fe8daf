// Hand-written HIP comparators for `kernelh bench` (backends hipref-naive,
// hipref-vec and the roofline_fma row), compiled for gfx950 and embedded in
// the kernelh CLI only: they are baselines to measure the templates against,
// not part of the product library.
//
// Symbols and raw-pointer ABIs follow the reference's comparator set
// (bench/refs/*.hip, launched by bench/harness/hipref_backend.cpp:95-276 and
// roofline.cpp:100-145), so results.csv rows line up:
//   softmax_naive / softmax_vec4      (x, y, int rows, int cols)       grid rows, block min(cols,256)
//   layernorm_naive / layernorm_vec4  (x, gamma, beta, y, rows, cols)  grid rows, block 256
//   fused_gelu_naive / fused_gelu_vec4 (x, y, int n)                   grid ceil(n/256), block 256
//   scan_pass1_naive / scan_pass1_vec4 (x, y, totals, int n, int t)    grid t = ceil(n/256), block 256
//   scan_totals_naive / scan_totals_vec4 (totals, y, int t, int n)     grid 1, block 256
//   gemm_tiled (a, b, c, int m, int n, int k)                          grid (n/32, m/32), block (32, 8)
//   roofline_fma (c, int n, int iters)                                 grid ceil(n/256), block 256
// The *_vec4 forms need 16-byte aligned buffers and cols (n) % 4 == 0.
//
// They are deliberately plain: one workgroup per row with LDS reductions,
// one element (or float4) per thread, a 32x32 LDS-tiled scalar GEMM. Each
// is checked for correctness against the fp64 oracle by the GPU tests.
#include "kh_device.h"

namespace {

constexpr float kEps = 1e-5f;

struct MaxOp {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct SumOp {
  __device__ float operator()(float a, float b) const { return a + b; }
};

// Workgroup-wide reduction (blockDim.x <= 1024): xor-shuffles inside each
// wave, then every thread folds the per-wave results from LDS. `part` is the
// caller's 16-float LDS scratch; the trailing barrier lets it be reused.
template <class Op>
__device__ float block_reduce(float v, Op op, float ident, float *part) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o, 64));
  const int nw = (blockDim.x + 63) / 64;
  if ((threadIdx.x & 63) == 0) part[threadIdx.x / 64] = v;
  __syncthreads();
  float r = ident;
  for (int w = 0; w < nw; ++w) r = op(r, part[w]);
  __syncthreads();
  return r;
}

// Inclusive scan over the workgroup (blockDim.x <= 1024, multiple of 64).
// Returns this thread's inclusive prefix; *total gets the workgroup sum.
__device__ float block_incl_scan(float v, float *part, float *total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x / 64, nw = blockDim.x / 64;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  if (lane == 63) part[w] = v;
  __syncthreads();
  float before = 0.0f, all = 0.0f;
  for (int i = 0; i < nw; ++i) {
    if (i < w) before += part[i];
    all += part[i];
  }
  __syncthreads();
  *total = all;
  return before + v;
}

__device__ __forceinline__ float gelu_chain(float x) {
  const float t = 1.5f * x + 0.5f;  // the fused affine op (a = 1.5, b = 0.5)
  const float z = 0.7978845608f * (t + 0.044715f * t * t * t);
  return 0.5f * t * (1.0f + tanhf(z));
}

}  // namespace

// ------------------------------------------------------------------ softmax

extern "C" __global__ void softmax_naive(const float *__restrict__ x, float *__restrict__ y, int rows, int cols) {
  __shared__ float part[16];
  const int r = blockIdx.x;
  if (r >= rows) return;
  const float *xr = x + (int64_t)r * cols;
  float *yr = y + (int64_t)r * cols;
  float m = -INFINITY;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) m = fmaxf(m, xr[c]);
  m = block_reduce(m, MaxOp{}, -INFINITY, part);
  float s = 0.0f;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) s += expf(xr[c] - m);
  const float inv = 1.0f / block_reduce(s, SumOp{}, 0.0f, part);
  for (int c = threadIdx.x; c < cols; c += blockDim.x) yr[c] = expf(xr[c] - m) * inv;
}

extern "C" __global__ void softmax_vec4(const float4 *__restrict__ x, float4 *__restrict__ y, int rows, int cols) {
  __shared__ float part[16];
  const int r = blockIdx.x;
  if (r >= rows) return;
  const int c4 = cols / 4;
  const float4 *xr = x + (int64_t)r * c4;
  float4 *yr = y + (int64_t)r * c4;
  float m = -INFINITY;
  for (int c = threadIdx.x; c < c4; c += blockDim.x) {
    const float4 v = xr[c];
    m = fmaxf(fmaxf(m, fmaxf(v.x, v.y)), fmaxf(v.z, v.w));
  }
  m = block_reduce(m, MaxOp{}, -INFINITY, part);
  float s = 0.0f;
  for (int c = threadIdx.x; c < c4; c += blockDim.x) {
    const float4 v = xr[c];
    s += (expf(v.x - m) + expf(v.y - m)) + (expf(v.z - m) + expf(v.w - m));
  }
  const float inv = 1.0f / block_reduce(s, SumOp{}, 0.0f, part);
  for (int c = threadIdx.x; c < c4; c += blockDim.x) {
    const float4 v = xr[c];
    yr[c] = make_float4(expf(v.x - m) * inv, expf(v.y - m) * inv, expf(v.z - m) * inv, expf(v.w - m) * inv);
  }
}

// ---------------------------------------------------------------- layernorm

extern "C" __global__ void layernorm_naive(const float *__restrict__ x, const float *__restrict__ gamma,
                                           const float *__restrict__ beta, float *__restrict__ y, int rows,
                                           int cols) {
  __shared__ float part[16];
  const int r = blockIdx.x;
  if (r >= rows) return;
  const float *xr = x + (int64_t)r * cols;
  float *yr = y + (int64_t)r * cols;
  float s = 0.0f;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) s += xr[c];
  const float mean = block_reduce(s, SumOp{}, 0.0f, part) / (float)cols;
  float q = 0.0f;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) {
    const float d = xr[c] - mean;
    q += d * d;
  }
  const float inv = rsqrtf(block_reduce(q, SumOp{}, 0.0f, part) / (float)cols + kEps);
  for (int c = threadIdx.x; c < cols; c += blockDim.x) yr[c] = (xr[c] - mean) * inv * gamma[c] + beta[c];
}

extern "C" __global__ void layernorm_vec4(const float4 *__restrict__ x, const float4 *__restrict__ gamma,
                                          const float4 *__restrict__ beta, float4 *__restrict__ y, int rows,
                                          int cols) {
  __shared__ float part[16];
  const int r = blockIdx.x;
  if (r >= rows) return;
  const int c4 = cols / 4;
  const float4 *xr = x + (int64_t)r * c4;
  float4 *yr = y + (int64_t)r * c4;
  float s = 0.0f;
  for (int c = threadIdx.x; c < c4; c += blockDim.x) {
    const float4 v = xr[c];
    s += (v.x + v.y) + (v.z + v.w);
  }
  const float mean = block_reduce(s, SumOp{}, 0.0f, part) / (float)cols;
  float q = 0.0f;
  for (int c = threadIdx.x; c < c4; c += blockDim.x) {
    const float4 v = xr[c];
    const float a = v.x - mean, b = v.y - mean, d = v.z - mean, e = v.w - mean;
    q += (a * a + b * b) + (d * d + e * e);
  }
  const float inv = rsqrtf(block_reduce(q, SumOp{}, 0.0f, part) / (float)cols + kEps);
  for (int c = threadIdx.x; c < c4; c += blockDim.x) {
    const float4 v = xr[c], g = gamma[c], b = beta[c];
    yr[c] = make_float4((v.x - mean) * inv * g.x + b.x, (v.y - mean) * inv * g.y + b.y,
                        (v.z - mean) * inv * g.z + b.z, (v.w - mean) * inv * g.w + b.w);
  }
}

// --------------------------------------------------------------- fused_gelu

extern "C" __global__ void fused_gelu_naive(const float *__restrict__ x, float *__restrict__ y, int n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = gelu_chain(x[i]);
}

extern "C" __global__ void fused_gelu_vec4(const float4 *__restrict__ x, float4 *__restrict__ y, int n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n / 4; i += stride) {
    const float4 v = x[i];
    y[i] = make_float4(gelu_chain(v.x), gelu_chain(v.y), gelu_chain(v.z), gelu_chain(v.w));
  }
}

// --------------------------------------------------------------------- scan
// Two passes. Pass 1: workgroup b scans its chunk (256 elements naive, 1024
// as float4 per thread vec4) into y and writes the chunk total to
// totals[b]; workgroups past the data write a zero total. Pass 2, one
// workgroup: an exclusive scan over the totals in 256-wide steps with a
// running carry, adding each chunk's offset to its elements of y.

extern "C" __global__ void scan_pass1_naive(const float *__restrict__ x, float *__restrict__ y,
                                            float *__restrict__ totals, int n, int t) {
  __shared__ float part[16];
  const int b = blockIdx.x;
  if (b >= t) return;
  const int64_t i = (int64_t)b * 256 + threadIdx.x;
  float total;
  const float incl = block_incl_scan(i < n ? x[i] : 0.0f, part, &total);
  if (i < n) y[i] = incl;
  if (threadIdx.x == 0) totals[b] = total;
}

extern "C" __global__ void scan_pass1_vec4(const float *__restrict__ x, float *__restrict__ y,
                                           float *__restrict__ totals, int n, int t) {
  __shared__ float part[16];
  const int b = blockIdx.x;
  if (b >= t) return;
  const int64_t base = (int64_t)b * 1024;
  if (base >= n) {
    if (threadIdx.x == 0) totals[b] = 0.0f;
    return;
  }
  const int64_t i = base + 4 * threadIdx.x;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (i + 3 < n) {
    v = *reinterpret_cast<const float4 *>(x + i);
  } else {
    v.x = i < n ? x[i] : 0.f;
    v.y = i + 1 < n ? x[i + 1] : 0.f;
    v.z = i + 2 < n ? x[i + 2] : 0.f;
  }
  const float s1 = v.x + v.y, s2 = s1 + v.z, s3 = s2 + v.w;
  float total;
  const float excl = block_incl_scan(s3, part, &total) - s3;
  const float4 o = make_float4(excl + v.x, excl + s1, excl + s2, excl + s3);
  if (i + 3 < n) {
    *reinterpret_cast<float4 *>(y + i) = o;
  } else {
    if (i < n) y[i] = o.x;
    if (i + 1 < n) y[i + 1] = o.y;
    if (i + 2 < n) y[i + 2] = o.z;
  }
  if (threadIdx.x == 0) totals[b] = total;
}

namespace {
__device__ void add_chunk_offsets(const float *__restrict__ totals, float *__restrict__ y, int t, int n, int chunk) {
  __shared__ float part[16];
  __shared__ float offs[256];
  float carry = 0.0f;
  for (int c0 = 0; c0 < t; c0 += 256) {
    const int c = c0 + threadIdx.x;
    const float v = (threadIdx.x < 256 && c < t) ? totals[c] : 0.0f;
    float total;
    const float incl = block_incl_scan(v, part, &total);
    if (threadIdx.x < 256) offs[threadIdx.x] = carry + incl - v;
    carry += total;
    __syncthreads();
    const int last = (t - c0) < 256 ? (t - c0) : 256;
    for (int64_t e = (int64_t)c0 * chunk + threadIdx.x; e < (int64_t)(c0 + last) * chunk && e < n;
         e += blockDim.x)
      y[e] += offs[e / chunk - c0];
    __syncthreads();
  }
}
}  // namespace

extern "C" __global__ void scan_totals_naive(const float *__restrict__ totals, float *__restrict__ y, int t, int n) {
  add_chunk_offsets(totals, y, t, n, 256);
}

extern "C" __global__ void scan_totals_vec4(const float *__restrict__ totals, float *__restrict__ y, int t, int n) {
  add_chunk_offsets(totals, y, t, n, 1024);
}

// --------------------------------------------------------------------- gemm
// C = A B (row-major): a 32x32 C tile per workgroup of 32x8 threads, each
// thread four rows (ty + 8i) of one column; 32-deep K steps staged in LDS,
// zero-filled past the matrix edges.

extern "C" __global__ void gemm_tiled(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ c,
                                      int m, int n, int k) {
  __shared__ float As[32][33];
  __shared__ float Bs[32][33];
  const int tx = threadIdx.x, ty = threadIdx.y;
  const int col = blockIdx.x * 32 + tx;
  const int row0 = blockIdx.y * 32;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < k; k0 += 32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = ty + 8 * i;
      As[r][tx] = (row0 + r < m && k0 + tx < k) ? a[(int64_t)(row0 + r) * k + k0 + tx] : 0.0f;
      Bs[r][tx] = (k0 + r < k && col < n) ? b[(int64_t)(k0 + r) * n + col] : 0.0f;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) {
      const float bv = Bs[kk][tx];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = fmaf(As[ty + 8 * i][kk], bv, acc[i]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = row0 + ty + 8 * i;
    if (r < m && col < n) c[(int64_t)r * n + col] = acc[i];
  }
}

// ------------------------------------------------------------ roofline_fma
// Vector-ALU fp32 FMA ceiling: each thread runs 8 independent FMA chains of
// iters/8 steps on its element (2 FLOP per FMA).

extern "C" __global__ void roofline_fma(float *__restrict__ c, int n, int iters) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float s = c[i];
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = s + (float)j;
    for (int r = 0; r < iters / 8; ++r) {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = fmaf(v[j], 0.999999f, 1e-7f);
    }
    c[i] = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  }
}
