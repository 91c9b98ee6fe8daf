// fp32 MFMA GEMM building blocks for gfx950, shared by the product kernels
// (gemm.hip: `gemm`, `gemm_mid`, `gemm_small`) and the tune candidates
// (gemm_tune.hip, used by `kernelh tune`). The design is described at the
// top of gemm.hip.
#pragma once

#include "kh_device.h"
#include "kh_tiles.h"

namespace khg {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kGroupM = 8;
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 buffer descriptor: 32-bit data format
constexpr uint32_t kOutside = 0x80000000u;

// Tile geometry for WTM x WTN accumulators per wave, BKT-deep slabs.
template <int WTM, int WTN, int BKT>
struct Tile {
  static constexpr int BK = BKT;
  static constexpr int LDA = BK + 4;       // A in LDS: [m][k], padded rows
  static constexpr int BM = 64 * WTM;      // rows of C per workgroup
  static constexpr int BN = 64 * WTN;      // columns of C per workgroup
  static constexpr int LDB = BN + 4;       // B in LDS: [k][n], padded rows
  static constexpr int AROW = BK / 4;      // float4 per A row
  static constexpr int NA = BM * BK / 4 / kThreads;  // A float4 per thread per slab
  static constexpr int NB = BK * BN / 4 / kThreads;  // B float4 per thread per slab
  static constexpr int BROW = BN / 4;      // float4 per B row
  static constexpr int A_STAGE = BM * LDA;
  static constexpr int B_STAGE = BK * LDB;
  static_assert(NA * kThreads * 4 == BM * BK && NB * kThreads * 4 == BK * BN,
                "a slab must split into whole float4s over the 256 threads");
  static_assert(BK % 8 == 0, "slabs are consumed in 8-deep chunks");
};

template <class T>
struct Slab {
  float4 a[T::NA];
  float4 b[T::NB];
};

__device__ __forceinline__ float4 load4(const float *__restrict__ P, int64_t row, int64_t col, int64_t ld,
                                        int64_t rows, int64_t cols, bool vec) {
  if (vec && row < rows && col + 3 < cols) return *reinterpret_cast<const float4 *>(P + row * ld + col);
  float t[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) t[q] = (row < rows && col + q < cols) ? P[row * ld + col + q] : 0.0f;
  return make_float4(t[0], t[1], t[2], t[3]);
}

// Generic slab load: any shape, stride and alignment (guarded per element).
// A: BK/4 lanes cover a row of the slab; B: BN/4 lanes cover a row of the tile.
template <class T>
__device__ __forceinline__ void load_slab(Slab<T> &s, const float *__restrict__ A, const float *__restrict__ B,
                                          int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t m0,
                                          int64_t n0, int64_t k0, bool a_vec, bool b_vec, int tid) {
#pragma unroll
  for (int i = 0; i < T::NA; ++i) {
    const int idx = tid + kThreads * i;
    s.a[i] = load4(A, m0 + idx / T::AROW, k0 + 4 * (idx % T::AROW), lda, M, K, a_vec);
  }
#pragma unroll
  for (int i = 0; i < T::NB; ++i) {
    const int idx = tid + kThreads * i;
    s.b[i] = load4(B, k0 + idx / T::BROW, n0 + 4 * (idx % T::BROW), ldb, K, N, b_vec);
  }
}

// Fast slab load for 16-byte aligned A and B with k and n multiples of 4:
// unconditional dwordx4 buffer loads. Each resource spans the slab's rows
// that exist (A: tile rows m0.. below M; B: slab rows k0.. below K), so
// rows past the matrix read 0 through the hardware range check; a float4
// past K (A) or N (B) is sent to an offset outside the resource and reads 0
// as well. No branches, 32-bit offsets.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const float *base, int64_t rows, int64_t ld) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, (int)(rows * ld * 4), kRsrcWord3);
}

__device__ __forceinline__ float4 as_float4(u32x4 u) {
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
}

template <class T>
__device__ __forceinline__ void load_slab_vec(Slab<T> &s, const float *__restrict__ A, const float *__restrict__ B,
                                              int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                              int64_t m0, int64_t n0, int64_t k0, int tid) {
  const __amdgpu_buffer_rsrc_t ra = rows_rsrc(A + m0 * lda, (M - m0) < T::BM ? (M - m0) : T::BM, lda);
  const __amdgpu_buffer_rsrc_t rb = rows_rsrc(B + k0 * ldb, (K - k0) < T::BK ? (K - k0) : T::BK, ldb);
#pragma unroll
  for (int i = 0; i < T::NA; ++i) {
    const int idx = tid + kThreads * i;
    const int ar = idx / T::AROW, ak = 4 * (idx % T::AROW);  // A: row in tile, k in slab
    const uint32_t aoff = (k0 + ak < K) ? (uint32_t)((ar * lda + k0 + ak) * 4) : kOutside;
    s.a[i] = as_float4(__builtin_amdgcn_raw_buffer_load_b128(ra, aoff, 0, 0));
  }
#pragma unroll
  for (int i = 0; i < T::NB; ++i) {
    const int idx = tid + kThreads * i;
    const int bk = idx / T::BROW, bn = 4 * (idx % T::BROW);  // B: k in slab, column in tile
    const uint32_t boff = (n0 + bn < N) ? (uint32_t)((bk * ldb + n0 + bn) * 4) : kOutside;
    s.b[i] = as_float4(__builtin_amdgcn_raw_buffer_load_b128(rb, boff, 0, 0));
  }
}

template <class T>
__device__ __forceinline__ void store_slab(const Slab<T> &s, float *__restrict__ As, float *__restrict__ Bs,
                                           int tid) {
#pragma unroll
  for (int i = 0; i < T::NA; ++i) {
    const int idx = tid + kThreads * i;
    *reinterpret_cast<float4 *>(As + (idx / T::AROW) * T::LDA + 4 * (idx % T::AROW)) = s.a[i];
  }
#pragma unroll
  for (int i = 0; i < T::NB; ++i) {
    const int idx = tid + kThreads * i;
    *reinterpret_cast<float4 *>(Bs + (idx / T::BROW) * T::LDB + 4 * (idx % T::BROW)) = s.b[i];
  }
}

template <int WTM, int WTN, class T>
__device__ __forceinline__ void compute_slab(v16f (&acc)[WTM][WTN], const float *__restrict__ As,
                                             const float *__restrict__ Bs, int wm, int wn, int lane) {
  const int r = lane & 31, h = lane >> 5;
#pragma unroll
  for (int c = 0; c < T::BK / 8; ++c) {
    float4 a[WTM];
    float b[WTN][4];
#pragma unroll
    for (int i = 0; i < WTM; ++i)
      a[i] = *reinterpret_cast<const float4 *>(As + (wm * 32 * WTM + i * 32 + r) * T::LDA + 8 * c + 4 * h);
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int s = 0; s < 4; ++s) b[j][s] = Bs[(8 * c + 4 * h + s) * T::LDB + wn * 32 * WTN + j * 32 + r];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int i = 0; i < WTM; ++i) {
        const float av = s == 0 ? a[i].x : s == 1 ? a[i].y : s == 2 ? a[i].z : a[i].w;
#pragma unroll
        for (int j = 0; j < WTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, b[j][s], acc[i][j], 0, 0, 0);
      }
    }
  }
}

// Launch index -> (tile row, tile column): XCD-contiguous, then grouped.
__device__ __forceinline__ void tile_coords(int64_t pid, int64_t tiles_m, int64_t tiles_n, bool xcd_remap,
                                            int64_t &tm, int64_t &tn) {
  const int64_t total = tiles_m * tiles_n;
  if (xcd_remap) pid = (pid & 7) * (total >> 3) + (pid >> 3);
  const int64_t width = kGroupM * tiles_n;
  const int64_t group = pid / width;
  const int64_t first_m = group * kGroupM;
  const int64_t gsz = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  tm = first_m + (pid % width) % gsz;
  tn = (pid % width) / gsz;
}

// One workgroup's loop over its tiles. VEC selects the fast slab loads.
// As, Bs: the two LDS stages, A_STAGE and B_STAGE floats apart. (Offsets
// from one base keep the pointers visibly in LDS for the compiler; an array
// of stage pointers would turn every LDS access into a flat one.)
template <int WTM, int WTN, int BKT, bool VEC, bool PRIO>
__device__ __forceinline__ void gemm_tiles(const float *__restrict__ Ap, const float *__restrict__ Bp,
                                           float *__restrict__ Cp, int64_t M, int64_t N, int64_t K, int64_t lda,
                                           int64_t ldb, int64_t ldc, bool a_vec, bool b_vec, float *As,
                                           float *Bs) {
  using T = Tile<WTM, WTN, BKT>;
  constexpr int BK = T::BK;
  const int tid = threadIdx.x;
  const int lane = kh::lane_id();
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int64_t tiles_m = (M + T::BM - 1) / T::BM, tiles_n = (N + T::BN - 1) / T::BN;
  const int64_t total = tiles_m * tiles_n;
  const int64_t nslabs = (K + BK - 1) / BK;
  const int64_t nblocks = (int64_t)gridDim.x * gridDim.y * gridDim.z;
  const int64_t bid = blockIdx.x + (int64_t)gridDim.x * (blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
  const bool xcd_remap = (nblocks == total) && ((total & 7) == 0);

  for (int64_t pid = bid; pid < total; pid += nblocks) {
    int64_t tm, tn;
    tile_coords(pid, tiles_m, tiles_n, xcd_remap, tm, tn);
    const int64_t m0 = tm * T::BM, n0 = tn * T::BN;

    v16f acc[WTM][WTN];
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
      for (int j = 0; j < WTN; ++j) acc[i][j] = v16f{};

    if (VEC) {
      Slab<T> s;
      load_slab_vec<T>(s, Ap, Bp, M, N, K, lda, ldb, m0, n0, 0, tid);
      store_slab<T>(s, As, Bs, tid);
      __syncthreads();
      for (int64_t ks = 0; ks < nslabs; ++ks) {
        const int cur = ks & 1;
        const bool more = ks + 1 < nslabs;
        if (more) load_slab_vec<T>(s, Ap, Bp, M, N, K, lda, ldb, m0, n0, (ks + 1) * BK, tid);
        if (PRIO) __builtin_amdgcn_s_setprio(1);
        compute_slab<WTM, WTN, T>(acc, As + cur * T::A_STAGE, Bs + cur * T::B_STAGE, wm, wn, lane);
        if (PRIO) __builtin_amdgcn_s_setprio(0);
        if (more) store_slab<T>(s, As + (cur ^ 1) * T::A_STAGE, Bs + (cur ^ 1) * T::B_STAGE, tid);
        __syncthreads();
      }
    } else {
      for (int64_t ks = 0; ks < nslabs; ++ks) {
        Slab<T> s;
        load_slab<T>(s, Ap, Bp, M, N, K, lda, ldb, m0, n0, ks * BK, a_vec, b_vec, tid);
        store_slab<T>(s, As, Bs, tid);
        __syncthreads();
        compute_slab<WTM, WTN, T>(acc, As, Bs, wm, wn, lane);
        __syncthreads();
      }
    }

    // Accumulator layout: lane l, register r -> row 8(r/4) + 4(l/32) + r%4,
    // column l%32 of the 32x32 block.
    const int col = lane & 31, h = lane >> 5;
#pragma unroll
    for (int i = 0; i < WTM; ++i) {
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        const int64_t gc = n0 + wn * 32 * WTN + j * 32 + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t gr = m0 + wm * 32 * WTM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          if (gr < M && gc < N) Cp[gr * ldc + gc] = acc[i][j][r];
        }
      }
    }
  }
}

template <int WTM, int WTN, int BKT, bool PRIO>
__device__ __forceinline__ void gemm_entry(const float *__restrict__ Ap, const float *__restrict__ Bp,
                                           float *__restrict__ Cp, int64_t M, int64_t N, int64_t K, int64_t lda,
                                           int64_t ldb, int64_t ldc) {
  using T = Tile<WTM, WTN, BKT>;
  __shared__ __attribute__((aligned(16))) float As[2 * T::A_STAGE];
  __shared__ __attribute__((aligned(16))) float Bs[2 * T::B_STAGE];
  const bool a_vec = ((K & 3) == 0) && ((lda & 3) == 0) && kh::aligned16(Ap);
  const bool b_vec = ((N & 3) == 0) && ((ldb & 3) == 0) && kh::aligned16(Bp);
  // The fast loads address a tile's rows with 32-bit byte offsets.
  const bool fits32 = (int64_t)T::BM * lda * 4 < (1ll << 31) && (int64_t)T::BK * ldb * 4 < (1ll << 31);
  if (a_vec && b_vec && fits32)
    gemm_tiles<WTM, WTN, BKT, true, PRIO>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, a_vec, b_vec, As, Bs);
  else
    gemm_tiles<WTM, WTN, BKT, false, PRIO>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, a_vec, b_vec, As, Bs);
}

}  // namespace khg
