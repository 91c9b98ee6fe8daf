// Layernorm over the last dim for gfx950, eps = 1e-5:
//   y = (x - mean) * rsqrt(var + eps) * gamma + beta.
//
// Symbol and memref arguments follow the reference template
// (lib/dsl/kernels/layernorm.cpp:58-153): x [rows, cols], gamma [cols],
// beta [cols], y [rows, cols], 24 parameters. Two-pass statistics as the
// template pins them (mean first, then the mean of squared deviations; no
// Welford), but the row is read from HBM once: one wavefront holds the row
// in registers (dwordx4 loads), so the second pass runs on registers. gamma
// and beta are read per row from L2 (every row shares them, so HBM sees them
// once). Traffic: 8 B per element + 8 B per column.
//
// Wider rows than the register path, unaligned or odd-width rows take a
// streaming form with the same two-pass statistics (the row is re-read from
// cache for the variance and the output). Rows are grid-strided over
// wavefronts; any block that is a multiple of 64 threads is correct,
// including the reference's rows x 256 geometry (kernelh_backend.cpp:290).
#include "kh_device.h"

#ifndef KH_LN_MAXV
#define KH_LN_MAXV 16  // float4 per lane on the register path: cols <= 4096
#endif

namespace {

constexpr float kEps = 1e-5f;

// gamma and beta are re-read per row from L2 (cols x 8 B, shared by every
// row) rather than held in registers: holding them doubled the register
// footprint and halved the number of rows in flight.
template <int V>
__device__ __forceinline__ void layernorm_rows_regs(const float *__restrict__ X, const float *__restrict__ G,
                                                    const float *__restrict__ B, float *__restrict__ Y,
                                                    int64_t rows, int64_t cols, int64_t xs, int64_t ys,
                                                    int64_t r0, int64_t rstep, int lane) {
  const float inv_cols = 1.0f / (float)cols;
  for (int64_t r = r0; r < rows; r += rstep) {
    const float *xr = X + r * xs;
    float *yr = Y + r * ys;
    float4 v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int64_t c = (int64_t)(lane + j * kh::kWave) * 4;
      v[j] = (c < cols) ? kh::load_nt(xr + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    const float mean = kh::wave_sum(s) * inv_cols;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int64_t c = (int64_t)(lane + j * kh::kWave) * 4;
      if (c < cols) {
        const float dx = v[j].x - mean, dy = v[j].y - mean, dz = v[j].z - mean, dw = v[j].w - mean;
        q += (dx * dx + dy * dy) + (dz * dz + dw * dw);
      }
    }
    const float var = kh::wave_sum(q) * inv_cols;
    const float inv = __builtin_amdgcn_rsqf(var + kEps);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int64_t c = (int64_t)(lane + j * kh::kWave) * 4;
      if (c < cols) {
        const float4 g = *reinterpret_cast<const float4 *>(G + c);
        const float4 b = *reinterpret_cast<const float4 *>(B + c);
        float4 o;
        o.x = fmaf((v[j].x - mean) * inv, g.x, b.x);
        o.y = fmaf((v[j].y - mean) * inv, g.y, b.y);
        o.z = fmaf((v[j].z - mean) * inv, g.z, b.z);
        o.w = fmaf((v[j].w - mean) * inv, g.w, b.w);
        kh::store_nt(yr + c, o);
      }
    }
  }
}

__device__ __forceinline__ void layernorm_row_stream(const float *__restrict__ xr, const float *__restrict__ G,
                                                     const float *__restrict__ B, float *__restrict__ yr,
                                                     int64_t cols, int lane) {
  float s = 0.0f;
  for (int64_t c = lane; c < cols; c += kh::kWave) s += xr[c];
  const float mean = kh::wave_sum(s) / (float)cols;
  float q = 0.0f;
  for (int64_t c = lane; c < cols; c += kh::kWave) {
    const float d = xr[c] - mean;
    q += d * d;
  }
  const float var = kh::wave_sum(q) / (float)cols;
  const float inv = __builtin_amdgcn_rsqf(var + kEps);
  for (int64_t c = lane; c < cols; c += kh::kWave) yr[c] = fmaf((xr[c] - mean) * inv, G[c], B[c]);
}

// Shared by both symbols; WIDE selects the register-path widths compiled in
// (the kernel's register allocation is that of its widest path).
template <bool WIDE>
__device__ __forceinline__ void layernorm_all(const float *__restrict__ X, const float *__restrict__ G,
                                              const float *__restrict__ B, float *__restrict__ Y, int64_t rows,
                                              int64_t cols, int64_t xs, int64_t ys) {
  const int lane = kh::lane_id();
  const int64_t waves_per_block = blockDim.x / kh::kWave;
  const int64_t r0 = blockIdx.x * waves_per_block + threadIdx.x / kh::kWave;
  const int64_t rstep = waves_per_block * gridDim.x;
  const bool vec = ((cols & 3) == 0) && ((xs & 3) == 0) && ((ys & 3) == 0) && kh::aligned16(X) &&
                   kh::aligned16(Y) && kh::aligned16(G) && kh::aligned16(B);
  const int64_t v4 = (cols + 255) / 256;
  if (!WIDE && vec && v4 <= 1) {
    layernorm_rows_regs<1>(X, G, B, Y, rows, cols, xs, ys, r0, rstep, lane);
  } else if (!WIDE && vec && v4 <= 2) {
    layernorm_rows_regs<2>(X, G, B, Y, rows, cols, xs, ys, r0, rstep, lane);
  } else if (!WIDE && vec && v4 <= 4) {
    layernorm_rows_regs<4>(X, G, B, Y, rows, cols, xs, ys, r0, rstep, lane);
  } else if (WIDE && vec && v4 <= 8) {
    layernorm_rows_regs<8>(X, G, B, Y, rows, cols, xs, ys, r0, rstep, lane);
  } else if (WIDE && vec && v4 <= KH_LN_MAXV) {
    layernorm_rows_regs<KH_LN_MAXV>(X, G, B, Y, rows, cols, xs, ys, r0, rstep, lane);
  } else {
    for (int64_t r = r0; r < rows; r += rstep) layernorm_row_stream(X + r * xs, G, B, Y + r * ys, cols, lane);
  }
}

}  // namespace

// The reference symbol: register path for rows up to 1024 floats, any other
// shape through the streaming path.
extern "C" __global__ void __launch_bounds__(256)
layernorm(KH_MEMREF2(const float, x), KH_MEMREF1(const float, gamma), KH_MEMREF1(const float, beta),
          KH_MEMREF2(float, y)) {
  layernorm_all<false>(KH_PTR(x), KH_PTR(gamma), KH_PTR(beta), KH_PTR(y), x_n0, x_n1, x_s0, y_s0);
}

// Same arguments and results; register path for rows of 1025..4096 floats
// (the launcher picks it for those widths).
extern "C" __global__ void __launch_bounds__(256)
layernorm_wide(KH_MEMREF2(const float, x), KH_MEMREF1(const float, gamma), KH_MEMREF1(const float, beta),
               KH_MEMREF2(float, y)) {
  layernorm_all<true>(KH_PTR(x), KH_PTR(gamma), KH_PTR(beta), KH_PTR(y), x_n0, x_n1, x_s0, y_s0);
}
