// Row-wise safe softmax for gfx950: y[r,:] = exp(x[r,:] - max) / sum.
//
// Symbol and memref arguments follow the reference template
// (lib/dsl/kernels/softmax.cpp:68-165): x, y rank-2 [rows, cols], 14
// parameters. The reference runs an online max/sum recurrence serially in
// every thread of a row's block (softmax.cpp:121-145), reading the row 256
// times. Here ONE wavefront owns a row: the row is read once with dwordx4
// loads into registers (cols <= 64 lanes x 4 x KH_SM_MAXV floats), reduced
// with DPP row rotations + readlane (max, then the sum of exponentials),
// and written once: 8 B of HBM traffic per element.
//
// Rows wider than the register path fall back to a two-sweep form (an online
// per-lane (max, sum) pass, then a write pass that re-reads the row). Rows
// are grid-strided over wavefronts; blocks that are not whole wavefronts
// give each thread whole rows instead, so every launch is correct, including
// the reference's rows x min(cols, 256) geometry (kernelh_backend.cpp:
// 256-257) at any cols.
//
// exp(x - m) is evaluated as 2^(x*log2e - m*log2e) with one fma on
// v_exp_f32; y = e * (1/s) with an IEEE reciprocal of s.
#include "kh_device.h"

#ifndef KH_SM_MAXV
#define KH_SM_MAXV 16  // float4 per lane on the register path: cols <= 4096
#endif

namespace {

// The row moves through buffer resources spanning exactly its cols floats:
// columns past the end read 0 (replaced by -inf before the max) and their
// stores are dropped, so the path has no per-lane branches. With SPLIT (a
// wave's first row in a launch that fits one round, four or more float4 per
// lane) the loads go out in two halves, the second once the first has
// landed, and nothing else is issued until all have (kh::kFirstBurst).
template <int V, bool SPLIT = false>
__device__ __forceinline__ void softmax_row_regs(const float *__restrict__ xr, float *__restrict__ yr,
                                                 int64_t cols, int lane) {
  const __amdgpu_buffer_rsrc_t rx = kh::span_rsrc(xr, (uint32_t)cols * 4u);
  const __amdgpu_buffer_rsrc_t ry = kh::span_rsrc(yr, (uint32_t)cols * 4u);
  constexpr int kHalf = V >= 4 ? V / 2 : V;
  float4 v[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    v[j] = kh::buf_load4_nt(rx, (uint32_t)(lane + j * kh::kWave) * 16u);
    if (SPLIT && j + 1 == kHalf && kHalf < V) kh::vm_wait<0>();
  }
  if (SPLIT) kh::vm_wait<0>();
  const float ninf = -__builtin_inff();
  float m = ninf;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    if ((int64_t)(lane + j * kh::kWave) * 4 >= cols) v[j] = make_float4(ninf, ninf, ninf, ninf);
    m = fmaxf(m, fmaxf(fmaxf(v[j].x, v[j].y), fmaxf(v[j].z, v[j].w)));
  }
  m = kh::wave_max(m);
  const float mb = -m * kh::kLog2e;
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    v[j].x = kh::exp2_hw(fmaf(v[j].x, kh::kLog2e, mb));
    v[j].y = kh::exp2_hw(fmaf(v[j].y, kh::kLog2e, mb));
    v[j].z = kh::exp2_hw(fmaf(v[j].z, kh::kLog2e, mb));
    v[j].w = kh::exp2_hw(fmaf(v[j].w, kh::kLog2e, mb));
    s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  }
  s = kh::wave_sum(s);
  const float inv = 1.0f / s;
#pragma unroll
  for (int j = 0; j < V; ++j)
    kh::buf_store4_nt(ry, (uint32_t)(lane + j * kh::kWave) * 16u,
                      make_float4(v[j].x * inv, v[j].y * inv, v[j].z * inv, v[j].w * inv));
}

// Any cols, any alignment: per-lane online (max, sum) over a strided sweep,
// merged across the wave, then a second sweep writes the outputs.
__device__ __forceinline__ void softmax_row_stream(const float *__restrict__ xr, float *__restrict__ yr,
                                                   int64_t cols, int lane) {
  float m = -__builtin_inff(), s = 0.0f;
  for (int64_t c = lane; c < cols; c += kh::kWave) {
    const float x = xr[c];
    const float mn = fmaxf(m, x);
    s = s * kh::exp2_hw((m - mn) * kh::kLog2e) + kh::exp2_hw((x - mn) * kh::kLog2e);
    m = mn;
  }
  const float gm = kh::wave_max(m);
  // Lanes that saw no element carry m = -inf, s = 0: contribute 0.
  s = (s == 0.0f) ? 0.0f : s * kh::exp2_hw((m - gm) * kh::kLog2e);
  const float gs = kh::wave_sum(s);
  const float inv = 1.0f / gs;
  const float mb = -gm * kh::kLog2e;
  for (int64_t c = lane; c < cols; c += kh::kWave) yr[c] = kh::exp2_hw(fmaf(xr[c], kh::kLog2e, mb)) * inv;
}

// Blocks that are not whole wavefronts (the reference's rows x
// min(cols, 256) geometry, kernelh_backend.cpp:256-257, when cols < 256 is
// not a multiple of 64): the wave reductions need 64 active lanes, so each
// thread takes whole rows, serially.
__device__ __forceinline__ void softmax_row_serial(const float *__restrict__ xr, float *__restrict__ yr,
                                                   int64_t cols) {
  float m = -__builtin_inff();
  for (int64_t c = 0; c < cols; ++c) m = fmaxf(m, xr[c]);
  const float mb = -m * kh::kLog2e;
  float s = 0.0f;
  for (int64_t c = 0; c < cols; ++c) s += kh::exp2_hw(fmaf(xr[c], kh::kLog2e, mb));
  const float inv = 1.0f / s;
  for (int64_t c = 0; c < cols; ++c) yr[c] = kh::exp2_hw(fmaf(xr[c], kh::kLog2e, mb)) * inv;
}

// Row loop shared by both symbols. WIDE selects which register-path widths
// are compiled in: the kernel's register allocation is that of its widest
// path, so the narrow symbol stays lean (more rows in flight per CU).
template <bool WIDE>
__device__ __forceinline__ void softmax_rows(const float *__restrict__ X, float *__restrict__ Y, int64_t rows,
                                             int64_t cols, int64_t xs, int64_t ys, int64_t bd, int64_t nb) {
  if (bd % kh::kWave != 0) {
    for (int64_t r = (int64_t)blockIdx.x * bd + threadIdx.x; r < rows; r += bd * nb)
      softmax_row_serial(X + r * xs, Y + r * ys, cols);
    return;
  }
  const int lane = kh::lane_id();
  const int64_t waves_per_block = bd / kh::kWave;
  const int64_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kh::kWave);  // uniform: scalar row loop
  const int64_t nwaves = waves_per_block * nb;
  const bool vec = ((cols & 3) == 0) && ((xs & 3) == 0) && ((ys & 3) == 0) && kh::aligned16(X) &&
                   kh::aligned16(Y);
  const int64_t v4 = (cols + 255) / 256;  // float4 per lane needed
  bool split = kh::split_first_burst(bd * nb);  // each wave's first row only
  for (int64_t r = blockIdx.x * waves_per_block + wave; r < rows; r += nwaves) {
    const float *xr = X + r * xs;
    float *yr = Y + r * ys;
    if (!WIDE && vec && v4 <= 1) {
      softmax_row_regs<1>(xr, yr, cols, lane);
    } else if (!WIDE && vec && v4 <= 2) {
      softmax_row_regs<2>(xr, yr, cols, lane);
    } else if (!WIDE && vec && v4 <= 4) {
      split ? softmax_row_regs<4, true>(xr, yr, cols, lane) : softmax_row_regs<4>(xr, yr, cols, lane);
    } else if (WIDE && vec && v4 <= 8) {
      split ? softmax_row_regs<8, true>(xr, yr, cols, lane) : softmax_row_regs<8>(xr, yr, cols, lane);
    } else if (WIDE && vec && v4 <= KH_SM_MAXV) {
      split ? softmax_row_regs<KH_SM_MAXV, true>(xr, yr, cols, lane) : softmax_row_regs<KH_SM_MAXV>(xr, yr, cols, lane);
    } else {
      softmax_row_stream(xr, yr, cols, lane);
    }
    split = false;
  }
}

}  // namespace

// The reference symbol: register path for rows up to 1024 floats, any other
// shape through the streaming path.
extern "C" __global__ void __launch_bounds__(256)
softmax(KH_MEMREF2(const float, x), KH_MEMREF2(float, y)) {
  const uint32_t gw = kh::group_size_word(), nb = kh::grid_blocks_x();
  KH_ARGS_READY(x_base, x_off, x_n0, x_n1, x_s0, y_base, y_off, y_s0, gw, nb);
  softmax_rows<false>(KH_PTR(x), KH_PTR(y), x_n0, x_n1, x_s0, y_s0, kh::threads_x_of(gw), nb);
}

// Same arguments and results; register path for rows of 1025..4096 floats
// (the launcher picks it for those widths).
extern "C" __global__ void __launch_bounds__(256)
softmax_wide(KH_MEMREF2(const float, x), KH_MEMREF2(float, y)) {
  const uint32_t gw = kh::group_size_word(), nb = kh::grid_blocks_x();
  KH_ARGS_READY(x_base, x_off, x_n0, x_n1, x_s0, y_base, y_off, y_s0, gw, nb);
  softmax_rows<true>(KH_PTR(x), KH_PTR(y), x_n0, x_n1, x_s0, y_s0, kh::threads_x_of(gw), nb);
}
