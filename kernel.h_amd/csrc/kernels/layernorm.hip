// Layernorm over the last dim for gfx950, eps = 1e-5:
//   y = (x - mean) * rsqrt(var + eps) * gamma + beta.
//
// Symbol and memref arguments follow the reference template
// (lib/dsl/kernels/layernorm.cpp:58-153): x [rows, cols], gamma [cols],
// beta [cols], y [rows, cols], 24 parameters. Two-pass statistics as the
// template pins them (mean first, then the mean of squared deviations; no
// Welford), but the row is read from HBM once: one wavefront holds the row
// in registers (dwordx4 loads), so the second pass runs on registers. Rows
// up to 1024 floats read gamma and beta once per workgroup into LDS; wider
// rows re-read them per row from L2. Every row shares them, so HBM sees them
// once either way. Traffic: 8 B per element + 8 B per column.
//
// Wider rows than the register path, unaligned or odd-width rows take a
// streaming form with the same two-pass statistics (the row is re-read from
// cache for the variance and the output). Rows are grid-strided over
// wavefronts; any block that is a multiple of 64 threads is correct,
// including the reference's rows x 256 geometry (kernelh_backend.cpp:290).
#include <type_traits>

#include "kh_device.h"

#ifndef KH_LN_MAXV
#define KH_LN_MAXV 16  // float4 per lane on the register path: cols <= 4096
#endif

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr float kEps = 1e-5f;

// Columns the narrow symbol stages gamma and beta for in LDS.
constexpr int kStageCols = 1024;

// gamma and beta (cols x 8 B, shared by every row) are not held in
// registers: that doubled the register footprint and halved the number of
// rows in flight. With STAGED (cols <= kStageCols) the workgroup copies them
// into Gs/Bs once, after its waves have issued their first row's loads, and
// the output reads them from LDS; otherwise each row re-reads them from L2.
// The LDS copy takes 4x fewer L2 requests for the same 64 lines, which every
// wave on the chip asks for at the same time. Measured at 4096x1024 it runs
// level with the L2 re-read (7.4-7.8 us) in a quiet sequence, but held
// 7.4-7.7 us in the first launches after a run of long GEMMs, where the L2
// re-read took 8.0-8.4 us.
// Rows move through buffer resources spanning exactly cols floats: columns
// past the end read 0 (kept out of the variance by a select) and their
// stores are dropped, so the path has no per-lane branches. For a wave's first
// staged row, in a launch that fits one round, and four or more float4 per
// lane, the loads go out in two halves, the second once the first has landed
// (kh::kFirstBurst). Without STAGED, gamma and beta are read
// the same way; with it, from LDS (a lane past cols reads a staged slot it
// does not use: every path that stages has 4 V float4 <= kStageCols).
template <int V, bool STAGED>
__device__ __forceinline__ void layernorm_rows_regs(const float *__restrict__ X, const float *__restrict__ G,
                                                    const float *__restrict__ B, float *__restrict__ Y,
                                                    int64_t rows, int64_t cols, int64_t xs, int64_t ys,
                                                    int64_t r0, int64_t rstep, int64_t bd, int lane, float *Gs,
                                                    float *Bs) {
  static_assert(!STAGED || 4 * V * kh::kWave <= kStageCols, "staged slots cover every lane's columns");
  const float inv_cols = 1.0f / (float)cols;
  const uint32_t row_bytes = (uint32_t)cols * 4u;
  constexpr int kHalf = V >= 4 ? V / 2 : V;
  float4 v[V];
  auto load_row = [&](int64_t r, auto split_tag) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rx = kh::span_rsrc(X + r * xs, row_bytes);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      v[j] = kh::buf_load4_nt(rx, (uint32_t)(lane + j * kh::kWave) * 16u);
      if (decltype(split_tag)::value && j + 1 == kHalf && kHalf < V) kh::vm_wait<0>();
    }
  };
  if constexpr (STAGED) {
    // Every thread of the block reaches the barrier: the staging sits
    // outside the row loop, and the path choice is uniform over the launch.
    // The first row's loads go out before the gamma/beta copy, whose LDS
    // writes wait for them as well (issue order).
    if (r0 < rows) {
      if (kh::split_first_burst(rstep * kh::kWave))  // launch threads
        load_row(r0, std::true_type{});
      else
        load_row(r0, std::false_type{});
    }
    for (int64_t i = threadIdx.x; 4 * i < cols; i += bd) {
      reinterpret_cast<float4 *>(Gs)[i] = reinterpret_cast<const float4 *>(G)[i];
      reinterpret_cast<float4 *>(Bs)[i] = reinterpret_cast<const float4 *>(B)[i];
    }
    kh::lds_barrier();
  }
  const __amdgpu_buffer_rsrc_t rg = kh::span_rsrc(G, row_bytes), rb = kh::span_rsrc(B, row_bytes);
  for (int64_t r = r0; r < rows; r += rstep) {
    const __amdgpu_buffer_rsrc_t ry = kh::span_rsrc(Y + r * ys, row_bytes);
    if (!STAGED || r != r0) load_row(r, std::false_type{});
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    const float mean = kh::wave_sum(s) * inv_cols;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float dx = v[j].x - mean, dy = v[j].y - mean, dz = v[j].z - mean, dw = v[j].w - mean;
      const float qj = (dx * dx + dy * dy) + (dz * dz + dw * dw);
      q += (int64_t)(lane + j * kh::kWave) * 4 < cols ? qj : 0.0f;
    }
    const float var = kh::wave_sum(q) * inv_cols;
    const float inv = __builtin_amdgcn_rsqf(var + kEps);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const uint32_t c = (uint32_t)(lane + j * kh::kWave) * 4u;
      float4 g, b;
      if constexpr (STAGED) {
        g = *reinterpret_cast<const float4 *>(Gs + c);
        b = *reinterpret_cast<const float4 *>(Bs + c);
      } else {
        const u32x4 gu = __builtin_amdgcn_raw_buffer_load_b128(rg, 4u * c, 0, 0);
        const u32x4 bu = __builtin_amdgcn_raw_buffer_load_b128(rb, 4u * c, 0, 0);
        g = make_float4(__uint_as_float(gu.x), __uint_as_float(gu.y), __uint_as_float(gu.z), __uint_as_float(gu.w));
        b = make_float4(__uint_as_float(bu.x), __uint_as_float(bu.y), __uint_as_float(bu.z), __uint_as_float(bu.w));
      }
      float4 o;
      o.x = fmaf((v[j].x - mean) * inv, g.x, b.x);
      o.y = fmaf((v[j].y - mean) * inv, g.y, b.y);
      o.z = fmaf((v[j].z - mean) * inv, g.z, b.z);
      o.w = fmaf((v[j].w - mean) * inv, g.w, b.w);
      kh::buf_store4_nt(ry, 4u * c, o);
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

// Blocks that are not whole wavefronts (the reference's own layernorm
// launches use 256 threads, but any block size is accepted): the wave
// reductions need 64 active lanes, so each thread takes whole rows,
// serially, with the same two-pass statistics.
__device__ __forceinline__ void layernorm_row_serial(const float *__restrict__ xr, const float *__restrict__ G,
                                                     const float *__restrict__ B, float *__restrict__ yr,
                                                     int64_t cols) {
  float s = 0.0f;
  for (int64_t c = 0; c < cols; ++c) s += xr[c];
  const float mean = s / (float)cols;
  float q = 0.0f;
  for (int64_t c = 0; c < cols; ++c) {
    const float d = xr[c] - mean;
    q += d * d;
  }
  const float inv = __builtin_amdgcn_rsqf(q / (float)cols + kEps);
  for (int64_t c = 0; c < cols; ++c) yr[c] = fmaf((xr[c] - mean) * inv, G[c], B[c]);
}

// Shared by both symbols; WIDE selects the register-path widths compiled in
// (the kernel's register allocation is that of its widest path). Gs and Bs
// hold kStageCols floats each in the narrow symbol and are unused (null) in
// the wide one.
template <bool WIDE>
__device__ __forceinline__ void layernorm_all(const float *__restrict__ X, const float *__restrict__ G,
                                              const float *__restrict__ B, float *__restrict__ Y, int64_t rows,
                                              int64_t cols, int64_t xs, int64_t ys, int64_t bd, int64_t nb,
                                              float *Gs, float *Bs) {
  if (bd % kh::kWave != 0) {  // uniform over the block: no thread reaches a barrier below
    for (int64_t r = (int64_t)blockIdx.x * bd + threadIdx.x; r < rows; r += bd * nb)
      layernorm_row_serial(X + r * xs, G, B, Y + r * ys, cols);
    return;
  }
  const int lane = kh::lane_id();
  const int64_t waves_per_block = bd / kh::kWave;
  // Uniform per wave (readfirstlane): the row loop and its buffer resources stay scalar.
  const int64_t r0 = blockIdx.x * waves_per_block + __builtin_amdgcn_readfirstlane(threadIdx.x / kh::kWave);
  const int64_t rstep = waves_per_block * nb;
  const bool vec = ((cols & 3) == 0) && ((xs & 3) == 0) && ((ys & 3) == 0) && kh::aligned16(X) &&
                   kh::aligned16(Y) && kh::aligned16(G) && kh::aligned16(B);
  const int64_t v4 = (cols + 255) / 256;
  static_assert(kStageCols == 4 * 4 * kh::kWave, "the narrow symbol stages every column its widest path holds");
  if (!WIDE && vec && v4 <= 1) {
    layernorm_rows_regs<1, true>(X, G, B, Y, rows, cols, xs, ys, r0, rstep, bd, lane, Gs, Bs);
  } else if (!WIDE && vec && v4 <= 2) {
    layernorm_rows_regs<2, true>(X, G, B, Y, rows, cols, xs, ys, r0, rstep, bd, lane, Gs, Bs);
  } else if (!WIDE && vec && v4 <= 4) {
    layernorm_rows_regs<4, true>(X, G, B, Y, rows, cols, xs, ys, r0, rstep, bd, lane, Gs, Bs);
  } else if (WIDE && vec && v4 <= 8) {
    layernorm_rows_regs<8, false>(X, G, B, Y, rows, cols, xs, ys, r0, rstep, bd, lane, nullptr, nullptr);
  } else if (WIDE && vec && v4 <= KH_LN_MAXV) {
    layernorm_rows_regs<KH_LN_MAXV, false>(X, G, B, Y, rows, cols, xs, ys, r0, rstep, bd, lane, nullptr, nullptr);
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
  __shared__ __attribute__((aligned(16))) float Gs[kStageCols];
  __shared__ __attribute__((aligned(16))) float Bs[kStageCols];
  const uint32_t gw = kh::group_size_word(), nb = kh::grid_blocks_x();
  KH_ARGS_READY(x_base, x_off, x_n0, x_n1, x_s0, gamma_base, gamma_off, beta_base, beta_off, y_base, y_off, y_s0,
                gw, nb);
  layernorm_all<false>(KH_PTR(x), KH_PTR(gamma), KH_PTR(beta), KH_PTR(y), x_n0, x_n1, x_s0, y_s0,
                       kh::threads_x_of(gw), nb, Gs, Bs);
}

// Same arguments and results; register path for rows of 1025..4096 floats
// (the launcher picks it for those widths).
extern "C" __global__ void __launch_bounds__(256)
layernorm_wide(KH_MEMREF2(const float, x), KH_MEMREF1(const float, gamma), KH_MEMREF1(const float, beta),
               KH_MEMREF2(float, y)) {
  const uint32_t gw = kh::group_size_word(), nb = kh::grid_blocks_x();
  KH_ARGS_READY(x_base, x_off, x_n0, x_n1, x_s0, gamma_base, gamma_off, beta_base, beta_off, y_base, y_off, y_s0,
                gw, nb);
  layernorm_all<true>(KH_PTR(x), KH_PTR(gamma), KH_PTR(beta), KH_PTR(y), x_n0, x_n1, x_s0, y_s0,
                      kh::threads_x_of(gw), nb, nullptr, nullptr);
}
