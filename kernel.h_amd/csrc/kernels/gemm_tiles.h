// fp32 MFMA GEMM building blocks for gfx950, shared by the product kernels
// (gemm.hip: `gemm`, `gemm_mid`, `gemm_small`, `gemm_small_pf2`, `gemm_wide`) and the tune candidates
// (gemm_tune.hip, used by `kernelh tune`). The design is described at the
// top of gemm.hip.
#pragma once

#include "kh_device.h"
#include "kh_tiles.h"

namespace khg {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // the product kernels' workgroup (2x2 waves)
constexpr int kGroupM = 8;
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 buffer descriptor: 32-bit data format
constexpr uint32_t kOutside = 0x80000000u;

// The two fp32 MFMA shapes. MF = 32: v_mfma_f32_32x32x2f32 (A: lane l holds
// A[l%32][l/32]; D: lane l, register r holds row 8(r/4) + 4(l/32) + r%4,
// column l%32), consumed in 8-deep chunks. MF = 16: v_mfma_f32_16x16x4f32
// (A[l%16][l/16]; D: row 4(l/16) + r, column l%16), in 16-deep chunks. Both
// run at the same rate; 16x16 holds a quarter of the accumulator per
// instruction, so the same wave tile takes four times the instructions.
template <int MF>
struct Mfma;
template <>
struct Mfma<32> {
  typedef v16f Acc;
  static constexpr int CK = 8;  // k per chunk: one ds_read_b128 of A per lane
};
template <>
struct Mfma<16> {
  typedef v4f Acc;
  static constexpr int CK = 16;
};

// Tile geometry for WTM x WTN MF x MF accumulators per wave, a WGM x WGN
// grid of waves per workgroup, BKT-deep slabs, and the LDS layout of one
// stage, which depends on how the stage is filled (DMA):
//
//   Register-staged (DMA false): A as [m][k] with rows padded by 4 floats
//   (one ds_read_b128 per lane delivers four k values, conflict-free) and B
//   as [k][n] with rows padded by 4 floats (a half-wave reads 32 consecutive
//   n with ds_read_b32). Fragment addresses are affine in the lane, so each
//   is one base register plus immediate offsets.
//
//   Direct-to-LDS (DMA true): a wave's load writes 64 float4s contiguously,
//   so rows cannot be padded inside one load. A is [m][k] unpadded with the
//   float4 holding k = 4Q..4Q+3 of row R at quad Q ^ aswz(R), an XOR swizzle
//   that keeps every 8-lane (128 B) and 16-lane (256 B) phase of the
//   fragment reads on distinct banks; B is [k][n] grouped by the RPI rows one
//   wave's 1 KiB load covers, groups padded by 4 floats (the two lane halves
//   of a fragment read, rows 4 apart, land on different banks).
template <int WTM, int WTN, int BKT, bool DMA, int WGM = 2, int WGN = 2, int MF = 32>
struct Tile {
  static constexpr int kMF = MF, kWTM = WTM, kWTN = WTN, kWGN = WGN;
  static constexpr int NT = 64 * WGM * WGN;  // threads per workgroup
  static constexpr int BK = BKT;
  static constexpr int BM = MF * WTM * WGM;  // rows of C per workgroup
  static constexpr int BN = MF * WTN * WGN;  // columns of C per workgroup
  static constexpr int QP = BK / 4;        // float4 per A row
  static constexpr int BROW = BN / 4;      // float4 per B row
  static constexpr int RPI = DMA ? (BROW >= 64 ? 1 : 64 / BROW) : 1;  // B rows per padded group
  static constexpr int LDA = DMA ? BK : BK + 4;
  static constexpr int LDG = RPI * BN + 4; // floats per padded group of B rows
  static constexpr int NA = BM * BK / 4 / NT;  // A float4 per thread per slab
  static constexpr int NB = BK * BN / 4 / NT;  // B float4 per thread per slab
  static constexpr int A_STAGE = BM * LDA;
  static constexpr int B_STAGE = (BK / RPI) * LDG;
  static constexpr int SWZ_SHIFT = QP == 2 ? 2 : QP == 4 ? 1 : 0;
  static_assert(NA * NT * 4 == BM * BK && NB * NT * 4 == BK * BN,
                "a slab must split into whole float4s over the workgroup's threads");
  static_assert(BK % Mfma<MF>::CK == 0 && (!DMA || QP <= 8), "slabs are consumed in whole chunks");
  static_assert(BROW <= 64 || BROW % 64 == 0, "a wave's B load covers whole rows");
  static_assert(BK % RPI == 0, "B row groups split the slab");
  __device__ static constexpr int aswz(int row) { return DMA ? ((row >> SWZ_SHIFT) ^ (row >> 3)) & (QP - 1) : 0; }
  // Float offset of A (row, logical quad q) and of B (row, column) in a stage.
  __device__ static constexpr int a_at(int row, int q) { return row * LDA + 4 * (q ^ aswz(row)); }
  __device__ static constexpr int b_at(int row, int col) { return (row / RPI) * LDG + (row % RPI) * BN + col; }
  static_assert(WGN > 0 && (WGN & (WGN - 1)) == 0, "a power-of-two wave grid width");
  __device__ static constexpr int wave_m(int wave) { return wave >> __builtin_ctz(WGN); }
  __device__ static constexpr int wave_n(int wave) { return wave & (WGN - 1); }
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
// A: QP lanes cover a row of the slab; B: BROW lanes cover a row of the tile.
template <class T>
__device__ __forceinline__ void load_slab(Slab<T> &s, const float *__restrict__ A, const float *__restrict__ B,
                                          int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t m0,
                                          int64_t n0, int64_t k0, bool a_vec, bool b_vec, int tid) {
#pragma unroll
  for (int i = 0; i < T::NA; ++i) {
    const int idx = tid + T::NT * i;
    s.a[i] = load4(A, m0 + idx / T::QP, k0 + 4 * (idx % T::QP), lda, M, K, a_vec);
  }
#pragma unroll
  for (int i = 0; i < T::NB; ++i) {
    const int idx = tid + T::NT * i;
    s.b[i] = load4(B, k0 + idx / T::BROW, n0 + 4 * (idx % T::BROW), ldb, K, N, b_vec);
  }
}

// Buffer resource over the slab rows that exist (A: tile rows m0.. below M;
// B: slab rows k0.. below K): rows past the matrix read 0 through the
// hardware range check; a float4 past K (A) or N (B) is sent to an offset
// outside the resource and reads 0 as well. 32-bit offsets.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const float *base, int64_t rows, int64_t ld) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, (int)(rows * ld * 4), kRsrcWord3);
}

// The same resource as four dwords, for the direct-to-LDS loads below.
__device__ __forceinline__ u32x4 rows_desc(const float *base, int64_t rows, int64_t ld) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  return u32x4{(uint32_t)b, (uint32_t)(b >> 32) & 0xffffu, (uint32_t)(rows * ld * 4), (uint32_t)kRsrcWord3};
}

__device__ __forceinline__ float4 as_float4(u32x4 u) {
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
}

// Register-staged slab load for 16-byte aligned A and B with k and n
// multiples of 4: unconditional dwordx4 buffer loads, no branches.
template <class T>
__device__ __forceinline__ void load_slab_vec(Slab<T> &s, const float *__restrict__ A, const float *__restrict__ B,
                                              int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                              int64_t m0, int64_t n0, int64_t k0, int tid) {
  const __amdgpu_buffer_rsrc_t ra = rows_rsrc(A + m0 * lda, (M - m0) < T::BM ? (M - m0) : T::BM, lda);
  const __amdgpu_buffer_rsrc_t rb = rows_rsrc(B + k0 * ldb, (K - k0) < T::BK ? (K - k0) : T::BK, ldb);
#pragma unroll
  for (int i = 0; i < T::NA; ++i) {
    const int idx = tid + T::NT * i;
    const int ar = idx / T::QP, ak = 4 * (idx % T::QP);  // A: row in tile, k in slab
    const uint32_t aoff = (k0 + ak < K) ? (uint32_t)((ar * lda + k0 + ak) * 4) : kOutside;
    s.a[i] = as_float4(__builtin_amdgcn_raw_buffer_load_b128(ra, aoff, 0, 0));
  }
#pragma unroll
  for (int i = 0; i < T::NB; ++i) {
    const int idx = tid + T::NT * i;
    const int bk = idx / T::BROW, bn = 4 * (idx % T::BROW);  // B: k in slab, column in tile
    const uint32_t boff = (n0 + bn < N) ? (uint32_t)((bk * ldb + n0 + bn) * 4) : kOutside;
    s.b[i] = as_float4(__builtin_amdgcn_raw_buffer_load_b128(rb, boff, 0, 0));
  }
}

// Register-staged (or generic) slab into LDS, in the tile's layout.
template <class T>
__device__ __forceinline__ void store_slab(const Slab<T> &s, float *__restrict__ As, float *__restrict__ Bs,
                                           int tid) {
#pragma unroll
  for (int i = 0; i < T::NA; ++i) {
    const int idx = tid + T::NT * i;
    *reinterpret_cast<float4 *>(As + T::a_at(idx / T::QP, idx % T::QP)) = s.a[i];
  }
#pragma unroll
  for (int i = 0; i < T::NB; ++i) {
    const int idx = tid + T::NT * i;
    *reinterpret_cast<float4 *>(Bs + T::b_at(idx / T::BROW, 4 * (idx % T::BROW))) = s.b[i];
  }
}

// One wave-wide direct-to-LDS float4 load (buffer_load_dwordx4 ... lds):
// lane l's 16 bytes from rsrc at byte offset voff land at LDS byte address
// lds + 16 l. M0 carries the LDS address; it is saved and restored around
// the load, with the one wait state the hardware needs between writing M0
// and an LDS-destination load. The load is inline assembly on purpose: the
// compiler cannot prove the LDS stages disjoint, and for its own form of
// this load it would wait for the load before every later LDS read. Here
// the caller orders it with vm_barrier.
__device__ __forceinline__ void dma16(u32x4 rsrc, uint32_t voff, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(voff), "s"(rsrc)
      : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const float *p) { return (uint32_t)reinterpret_cast<uintptr_t>(p); }

// Direct-to-LDS slab load for 16-byte aligned A and B with k and n multiples
// of 4. Each wave's instruction lands 64 float4s contiguously, so the lane ->
// global mapping realises the layout: in A, lane l of a wave fills physical
// quad l % QP of its row and so fetches logical quad (l % QP) ^ aswz(row); B
// is row-major within a group. Callers fetch slabs with k0 < K (or k0 = 0
// when K = 0, which reads nothing). `wave` must be wave-uniform.
//
// ALN (K a multiple of BK, N of BN): no float4 of a slab reaches past K or
// N, so the per-load tail selects go and each offset is a loop-invariant
// 32-bit term plus a wave-uniform one (k0 for A, n0 for B), which keeps the
// offsets of every load of a slab in registers even where the tile's
// accumulators leave few (rows past M still read 0 through the resource).
//
// dma_part issues loads L0..L1-1 of a slab (A's NA, then B's NB), so that a
// slab's loads can be spread between MFMAs; dma_slab issues all of them.
template <class T, bool ALN, int L0, int L1>
__device__ __forceinline__ void dma_part(const float *__restrict__ A, const float *__restrict__ B, int64_t M,
                                         int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t m0, int64_t n0,
                                         int64_t k0, float *As, float *Bs, int wave, int lane) {
  const u32x4 ra = rows_desc(A + m0 * lda, (M - m0) < T::BM ? (M - m0) : T::BM, lda);
  const u32x4 rb = rows_desc(B + k0 * ldb, (K - k0) < T::BK ? (K - k0) : T::BK, ldb);
#pragma unroll
  for (int i = 0; i < T::NA; ++i) {
    if (i < L0 || i >= L1) continue;
    const int idx0 = 64 * wave + T::NT * i;  // first float4 of this wave's instruction
    const int idx = idx0 + lane;
    const int ar = idx / T::QP, ak = 4 * ((idx % T::QP) ^ T::aswz(ar));
    uint32_t aoff;
    if constexpr (ALN)
      aoff = ((uint32_t)ar * (uint32_t)lda + (uint32_t)ak) * 4u + (uint32_t)k0 * 4u;
    else
      aoff = (k0 + ak < K) ? (uint32_t)((ar * lda + k0 + ak) * 4) : kOutside;
    dma16(ra, aoff, lds_addr(As + 4 * idx0));
  }
#pragma unroll
  for (int i = 0; i < T::NB; ++i) {
    if (T::NA + i < L0 || T::NA + i >= L1) continue;
    const int idx0 = 64 * wave + T::NT * i;
    const int idx = idx0 + lane;
    const int bk = idx / T::BROW, bn = 4 * (idx % T::BROW);
    uint32_t boff;
    if constexpr (ALN)
      boff = ((uint32_t)bk * (uint32_t)ldb + (uint32_t)bn) * 4u + (uint32_t)n0 * 4u;
    else
      boff = (n0 + bn < N) ? (uint32_t)((bk * ldb + n0 + bn) * 4) : kOutside;
    dma16(rb, boff, lds_addr(Bs + T::b_at(idx0 / T::BROW, 4 * (idx0 % T::BROW))));
  }
}

template <class T, bool ALN = false>
__device__ __forceinline__ void dma_slab(const float *__restrict__ A, const float *__restrict__ B, int64_t M,
                                         int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t m0, int64_t n0,
                                         int64_t k0, float *As, float *Bs, int wave, int lane) {
  dma_part<T, ALN, 0, T::NA + T::NB>(A, B, M, N, K, lda, ldb, m0, n0, k0, As, Bs, wave, lane);
}

// Wait until at most N vector-memory operations of this wave are in flight
// and all its LDS operations are done, then meet the workgroup. Loads retire
// in order, so N = the loads issued after the ones awaited. The wait is the
// s_waitcnt builtin, so the compiler's own bookkeeping knows that LDS reads
// issued before it are complete; the empty asm before it and the barrier
// asm after it (both memory clobbers) keep every LDS access on its side.
template <int N>
__device__ __forceinline__ void vm_barrier() {
  // 63 is the field's "do not wait" encoding, so the largest real wait is 62.
  static_assert(N >= 0 && N < 63, "vmcnt field");
  // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14].
  constexpr int kImm = (N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kImm);
  asm volatile("s_barrier" ::: "memory");
}

// Fragments of chunk c of a stage. The MFMA sums k over its lane groups,
// and any permutation of k applied to both operands gives the same product:
//   MF = 32 (8-deep chunks): lane half h takes k = 8c + 4h + {0..3} (one
//     ds_read_b128 for A); MFMA step s consumes k = 8c + s (half 0) and
//     8c + 4 + s (half 1).
//   MF = 16 (16-deep chunks): lane group g = l/16 takes quad q(g) =
//     (g%2)*2 + g/2, i.e. k = 16c + 4q + {0..3}; step s consumes
//     k = 16c + 4q(g) + s from group g. The order 0, 2, 1, 3 puts the B rows
//     that lanes 0-31 read in one step 8 apart, which keeps them on distinct
//     LDS banks in the direct-to-LDS layout, where two B rows share a group.
template <int WTM, int WTN>
struct Frag {
  float4 a[WTM];
  float b[WTN][4];
};

template <class T>
using AccOf = typename Mfma<T::kMF>::Acc;

template <int WTM, int WTN, class T>
__device__ __forceinline__ void read_frag(Frag<WTM, WTN> &f, const float *__restrict__ As, const float *__restrict__ Bs,
                                          int c, int wm, int wn, int lane) {
  if constexpr (T::kMF == 32) {
    const int r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int i = 0; i < WTM; ++i)
      f.a[i] = *reinterpret_cast<const float4 *>(As + T::a_at(wm * 32 * WTM + i * 32 + r, 2 * c + h));
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int s = 0; s < 4; ++s) f.b[j][s] = Bs[T::b_at(8 * c + 4 * h + s, wn * 32 * WTN + j * 32 + r)];
  } else {
    const int r = lane & 15, g = lane >> 4, q = ((g & 1) << 1) | (g >> 1);
#pragma unroll
    for (int i = 0; i < WTM; ++i)
      f.a[i] = *reinterpret_cast<const float4 *>(As + T::a_at(wm * 16 * WTM + i * 16 + r, 4 * c + q));
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int s = 0; s < 4; ++s) f.b[j][s] = Bs[T::b_at(16 * c + 4 * q + s, wn * 16 * WTN + j * 16 + r)];
  }
}

// MFMA steps S0..S1-1 of a chunk: a chunk's four steps can be split around
// other work, each accumulator still taking its steps in order (the same
// bits).
template <int WTM, int WTN, int S0, int S1, class Acc>
__device__ __forceinline__ void mfma_frag_s(Acc (&acc)[WTM][WTN], const Frag<WTM, WTN> &f) {
#pragma unroll
  for (int s = S0; s < S1; ++s)
#pragma unroll
    for (int i = 0; i < WTM; ++i) {
      const float av = s == 0 ? f.a[i].x : s == 1 ? f.a[i].y : s == 2 ? f.a[i].z : f.a[i].w;
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        if constexpr (sizeof(Acc) == sizeof(v16f))
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, f.b[j][s], acc[i][j], 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, f.b[j][s], acc[i][j], 0, 0, 0);
      }
    }
}

template <int WTM, int WTN, class Acc>
__device__ __forceinline__ void mfma_frag(Acc (&acc)[WTM][WTN], const Frag<WTM, WTN> &f) {
  mfma_frag_s<WTM, WTN, 0, 4>(acc, f);
}

// One slab's chunks from LDS (the register-staged pipelines). For eight-wave
// tiles on 16x16 MFMAs (the tune space's; `gemm_wide` was one before it
// moved to the persistent ring), chunk c+1's fragment reads are interleaved
// with chunk c's MFMAs, one read per two (kernel trace, variants
// interleaved launch by launch, same bits: 2048^3 142.5 -> 141.3 us,
// 6144x6144x1024 593.8 -> 586.1). The same change slowed the four-wave
// tiles (the then four-wave `gemm_small` 8-10%, `gemm_mid` 0.5-1%), which
// keep one chunk's reads before its MFMAs.
template <int WTM, int WTN, class T>
__device__ __forceinline__ void compute_slab(AccOf<T> (&acc)[WTM][WTN], const float *__restrict__ As,
                                             const float *__restrict__ Bs, int wm, int wn, int lane) {
  constexpr int C = T::BK / Mfma<T::kMF>::CK;
  if constexpr (T::NT == 512 && T::kMF == 16) {
    Frag<WTM, WTN> f[2];
    read_frag<WTM, WTN, T>(f[0], As, Bs, 0, wm, wn, lane);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (c + 1 < C) read_frag<WTM, WTN, T>(f[(c + 1) & 1], As, Bs, c + 1, wm, wn, lane);
      mfma_frag<WTM, WTN>(acc, f[c & 1]);
      if (c + 1 < C) {
#pragma unroll
        for (int g = 0; g < WTM + 2 * WTN; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two MFMAs
        }
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      Frag<WTM, WTN> f;
      read_frag<WTM, WTN, T>(f, As, Bs, c, wm, wn, lane);
      mfma_frag<WTM, WTN>(acc, f);
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

// Pipelines over the K slabs of one tile, accumulating into acc.
//
// DMA (direct-to-LDS, three stages; slab j in stage j % 3): the barrier sits
// after each slab's first 8-deep chunk. Once it passes, slab ks+1 has landed
// and every wave is done with slab ks-1, so slab ks+2's loads go into ks-1's
// stage and slab ks+1's first fragments are read while this slab's later
// chunks, already in registers, feed the MFMAs: no wave waits on LDS data
// right after a barrier, and each slab has one slab-time to arrive.
template <int WTM, int WTN, class T, bool PRIO>
__device__ __forceinline__ void k_loop_dma(AccOf<T> (&acc)[WTM][WTN], const float *__restrict__ Ap,
                                           const float *__restrict__ Bp, int64_t M, int64_t N, int64_t K,
                                           int64_t lda, int64_t ldb, int64_t m0, int64_t n0, int64_t nslabs,
                                           float *As, float *Bs, int wave, int wm, int wn, int lane) {
  constexpr int BK = T::BK;
  constexpr int C = BK / Mfma<T::kMF>::CK;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  dma_slab<T>(Ap, Bp, M, N, K, lda, ldb, m0, n0, 0, As, Bs, wv, lane);
  if (nslabs > 1) {
    dma_slab<T>(Ap, Bp, M, N, K, lda, ldb, m0, n0, BK, As + T::A_STAGE, Bs + T::B_STAGE, wv, lane);
    vm_barrier<T::NA + T::NB>();
  } else {
    vm_barrier<0>();
  }
  Frag<WTM, WTN> f0, f1;
  read_frag<WTM, WTN, T>(f0, As, Bs, 0, wm, wn, lane);
  int cur = 0;
  for (int64_t ks = 0; ks < nslabs; ++ks) {
    const int nxt = cur == 2 ? 0 : cur + 1;
    const int fut = nxt == 2 ? 0 : nxt + 1;
    const float *sA = As + cur * T::A_STAGE, *sB = Bs + cur * T::B_STAGE;
    if constexpr (C > 1) read_frag<WTM, WTN, T>(f1, sA, sB, 1, wm, wn, lane);
    if (PRIO) __builtin_amdgcn_s_setprio(1);
    mfma_frag<WTM, WTN>(acc, f0);
    if (PRIO) __builtin_amdgcn_s_setprio(0);
    vm_barrier<0>();
    if (ks + 2 < nslabs)
      dma_slab<T>(Ap, Bp, M, N, K, lda, ldb, m0, n0, (ks + 2) * BK, As + fut * T::A_STAGE, Bs + fut * T::B_STAGE,
                  wv, lane);
    if (ks + 1 < nslabs) read_frag<WTM, WTN, T>(f0, As + nxt * T::A_STAGE, Bs + nxt * T::B_STAGE, 0, wm, wn, lane);
    if (PRIO) __builtin_amdgcn_s_setprio(1);
    if constexpr (C > 1) mfma_frag<WTM, WTN>(acc, f1);
#pragma unroll
    for (int c = 2; c < C; ++c) {
      read_frag<WTM, WTN, T>(f1, sA, sB, c, wm, wn, lane);
      mfma_frag<WTM, WTN>(acc, f1);
    }
    if (PRIO) __builtin_amdgcn_s_setprio(0);
    cur = nxt;
  }
  // The next tile's first loads reuse stages 0 and 1.
  vm_barrier<0>();
}

// Register-staged (two stages): the next slab's global loads are in flight
// while the current slab feeds the MFMAs, one barrier per slab.
template <int WTM, int WTN, class T, bool PRIO>
__device__ __forceinline__ void k_loop_regs(AccOf<T> (&acc)[WTM][WTN], const float *__restrict__ Ap,
                                            const float *__restrict__ Bp, int64_t M, int64_t N, int64_t K,
                                            int64_t lda, int64_t ldb, int64_t m0, int64_t n0, int64_t nslabs,
                                            float *As, float *Bs, int tid, int wm, int wn, int lane) {
  Slab<T> s;
  load_slab_vec<T>(s, Ap, Bp, M, N, K, lda, ldb, m0, n0, 0, tid);
  store_slab<T>(s, As, Bs, tid);
  __syncthreads();
  for (int64_t ks = 0; ks < nslabs; ++ks) {
    const int cur = ks & 1;
    const bool more = ks + 1 < nslabs;
    if (more) load_slab_vec<T>(s, Ap, Bp, M, N, K, lda, ldb, m0, n0, (ks + 1) * T::BK, tid);
    if (PRIO) __builtin_amdgcn_s_setprio(1);
    compute_slab<WTM, WTN, T>(acc, As + cur * T::A_STAGE, Bs + cur * T::B_STAGE, wm, wn, lane);
    if (PRIO) __builtin_amdgcn_s_setprio(0);
    if (more) store_slab<T>(s, As + (cur ^ 1) * T::A_STAGE, Bs + (cur ^ 1) * T::B_STAGE, tid);
    __syncthreads();
  }
}

// Register-staged with two staging sets: slab ks+2's global loads are in
// flight while slab ks computes and slab ks+1 goes to LDS, so each load has
// two slab-times to arrive. The barriers fence LDS only (a full
// __syncthreads() would wait for those loads). The loop is unrolled by two
// so the staging sets swap roles without copies.
template <int WTM, int WTN, class T, bool PRIO>
__device__ __forceinline__ void prefetch2_step(AccOf<T> (&acc)[WTM][WTN], Slab<T> &free_set, Slab<T> &next_set,
                                               const float *__restrict__ Ap, const float *__restrict__ Bp,
                                               int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                               int64_t m0, int64_t n0, int64_t nslabs, int64_t ks, float *As,
                                               float *Bs, int tid, int wm, int wn, int lane) {
  const int cur = ks & 1;
  if (ks + 2 < nslabs) load_slab_vec<T>(free_set, Ap, Bp, M, N, K, lda, ldb, m0, n0, (ks + 2) * T::BK, tid);
  if (PRIO) __builtin_amdgcn_s_setprio(1);
  compute_slab<WTM, WTN, T>(acc, As + cur * T::A_STAGE, Bs + cur * T::B_STAGE, wm, wn, lane);
  if (PRIO) __builtin_amdgcn_s_setprio(0);
  if (ks + 1 < nslabs) store_slab<T>(next_set, As + (cur ^ 1) * T::A_STAGE, Bs + (cur ^ 1) * T::B_STAGE, tid);
  kh::lds_barrier();
}

template <int WTM, int WTN, class T, bool PRIO>
__device__ __forceinline__ void k_loop_prefetch2(AccOf<T> (&acc)[WTM][WTN], const float *__restrict__ Ap,
                                                 const float *__restrict__ Bp, int64_t M, int64_t N, int64_t K,
                                                 int64_t lda, int64_t ldb, int64_t m0, int64_t n0, int64_t nslabs,
                                                 float *As, float *Bs, int tid, int wm, int wn, int lane) {
  Slab<T> s0, s1;
  load_slab_vec<T>(s0, Ap, Bp, M, N, K, lda, ldb, m0, n0, 0, tid);
  if (nslabs > 1) load_slab_vec<T>(s1, Ap, Bp, M, N, K, lda, ldb, m0, n0, T::BK, tid);
  store_slab<T>(s0, As, Bs, tid);
  kh::lds_barrier();
  for (int64_t ks = 0; ks < nslabs; ks += 2) {
    prefetch2_step<WTM, WTN, T, PRIO>(acc, s0, s1, Ap, Bp, M, N, K, lda, ldb, m0, n0, nslabs, ks, As, Bs, tid, wm,
                                      wn, lane);
    if (ks + 1 < nslabs)
      prefetch2_step<WTM, WTN, T, PRIO>(acc, s1, s0, Ap, Bp, M, N, K, lda, ldb, m0, n0, nslabs, ks + 1, As, Bs,
                                        tid, wm, wn, lane);
  }
}

// Generic (any shape, stride, alignment): synchronous, one stage.
template <int WTM, int WTN, class T>
__device__ __forceinline__ void k_loop_generic(AccOf<T> (&acc)[WTM][WTN], const float *__restrict__ Ap,
                                               const float *__restrict__ Bp, int64_t M, int64_t N, int64_t K,
                                               int64_t lda, int64_t ldb, int64_t m0, int64_t n0, int64_t nslabs,
                                               bool a_vec, bool b_vec, float *As, float *Bs, int tid, int wm, int wn,
                                               int lane) {
  for (int64_t ks = 0; ks < nslabs; ++ks) {
    Slab<T> s;
    load_slab<T>(s, Ap, Bp, M, N, K, lda, ldb, m0, n0, ks * T::BK, a_vec, b_vec, tid);
    store_slab<T>(s, As, Bs, tid);
    __syncthreads();
    compute_slab<WTM, WTN, T>(acc, As, Bs, wm, wn, lane);
    __syncthreads();
  }
}

// Writes a tile's accumulators to C. Accumulator layout (MF = 32): lane l,
// register r -> row 8(r/4) + 4(l/32) + r%4, column l%32 of the 32x32 block,
// so each store instruction writes two 128-byte row pieces (whole cache
// lines); MF = 16: row 4(l/16) + r, column l%16, four 64-byte pieces.
template <int WTM, int WTN, class T>
__device__ __forceinline__ void store_tile(const AccOf<T> (&acc)[WTM][WTN], float *__restrict__ Cp, int64_t M,
                                           int64_t N, int64_t ldc, int64_t m0, int64_t n0, int wm, int wn,
                                           int lane) {
  constexpr int MF = T::kMF;
  const int col = lane & (MF - 1), h = lane / MF;
#pragma unroll
  for (int i = 0; i < WTM; ++i) {
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
      const int64_t gc = n0 + wn * MF * WTN + j * MF + col;
      if constexpr (MF == 32) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t gr = m0 + wm * 32 * WTM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          if (gr < M && gc < N) Cp[gr * ldc + gc] = acc[i][j][r];
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t gr = m0 + wm * 16 * WTM + i * 16 + 4 * h + r;
          if (gr < M && gc < N) Cp[gr * ldc + gc] = acc[i][j][r];
        }
      }
    }
  }
}

// Every kernel argument a GEMM entry uses, with the launch's block counts,
// loaded in one round before anything else (KH_ARGS_READY): the tile loops
// read the same words again, and those loads fold into these.
#define KH_GEMM_ARGS_READY(...)                                                                               \
  KH_ARGS_READY(A_base, A_off, A_n0, A_n1, A_s0, B_base, B_off, B_n1, B_s0, C_base, C_off, C_n0, C_n1, C_s0,  \
                kh::grid_blocks_x(), kh::grid_blocks_y(), kh::grid_blocks_z(), ##__VA_ARGS__)

// Writes NaN over C (grid-strided over the whole launch): how a kernel whose
// tile split assumes one workgroup size refuses a launch with another,
// instead of computing part of each tile.
__device__ __forceinline__ void refuse_launch(float *C, int64_t M, int64_t N, int64_t ldc) {
  const uint32_t gxy = kh::group_size_word();
  const int64_t tx = kh::threads_x_of(gxy), ty = kh::threads_y_of(gxy), tz = kh::threads_z_of(kh::group_size_z_word());
  const int64_t gx = kh::grid_blocks_x(), gy = kh::grid_blocks_y(), gz = kh::grid_blocks_z();
  const int64_t threads = tx * ty * tz;
  const int64_t flat = ((int64_t)threadIdx.z * ty + threadIdx.y) * tx + threadIdx.x;
  const int64_t block = ((int64_t)blockIdx.z * gy + blockIdx.y) * gx + blockIdx.x;
  const int64_t stride = gx * gy * gz * threads;
  for (int64_t i = block * threads + flat; i < M * N; i += stride) C[(i / N) * ldc + i % N] = __builtin_nanf("");
}

// store_tile for the persistent pipeline: buffer stores over a resource
// spanning the tile's rows inside C, so rows past M are dropped by the
// hardware range check and columns past N go to an offset outside it. Every
// lane issues exactly WTM x WTN x (16 or 4: the accumulator registers of one
// 32x32 or 16x16 block) store instructions, no branches,
// so a later wait can count them (gemm_tiles_flat waits for the next
// tile's slab loads while the most recent 62 of these stores stay in
// flight). Needs BM x ldc x 4 < 2^31.
template <int WTM, int WTN, class T>
__device__ __forceinline__ void store_tile_buf(const AccOf<T> (&acc)[WTM][WTN], float *__restrict__ Cp, int64_t M,
                                               int64_t N, int64_t ldc, int64_t m0, int64_t n0, int wm, int wn,
                                               int lane) {
  // Accumulator layouts: MF = 32, lane l, register r holds row
  // 8(r/4) + 4(l/32) + r%4 of its block; MF = 16, row 4(l/16) + r; column
  // l % MF in both.
  constexpr int MF = T::kMF;
  constexpr int kRegs = MF == 32 ? 16 : 4;
  const int64_t rows = (M - m0) < T::BM ? (M - m0) : T::BM;
  const __amdgpu_buffer_rsrc_t rc =
      __builtin_amdgcn_make_buffer_rsrc(Cp + m0 * ldc, (short)0, (int)(rows * ldc * 4), kRsrcWord3);
  const int col = lane & (MF - 1), h = lane / MF;
  const uint32_t ld4 = (uint32_t)ldc * 4u;
  // Per lane: one offset per column block (kOutside past N), plus each
  // store's row displacement. The displacement goes into the vector offset,
  // not the scalar one: the range check that drops rows past M covers the
  // vector offset (kOutside + a displacement below 2^31 stays out of range).
  uint32_t base[WTN];
#pragma unroll
  for (int j = 0; j < WTN; ++j) {
    const int gc = wn * MF * WTN + j * MF + col;
    base[j] = (n0 + gc < N) ? (uint32_t)((wm * MF * WTM + 4 * h) * ld4 + (uint32_t)(n0 + gc) * 4u) : kOutside;
  }
#pragma unroll
  for (int i = 0; i < WTM; ++i) {
#pragma unroll
    for (int r = 0; r < kRegs; ++r) {
      const int row = MF == 32 ? i * 32 + 8 * (r >> 2) + (r & 3) : i * 16 + r;
      const uint32_t rowoff = (uint32_t)row * ld4;
#pragma unroll
      for (int j = 0; j < WTN; ++j)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][r]), rc, base[j] + rowoff, 0, 0);
    }
  }
}

// Fast-path pipelines (gemm_body's PIPE).
constexpr int kPipeRegs = 1;       // register-staged, one slab ahead
constexpr int kPipeDma = 2;        // direct-to-LDS, three stages
constexpr int kPipePrefetch2 = 3;  // register-staged, two slabs ahead

// One workgroup's loop over its tiles. PATH: 0 generic, else a kPipe*. As, Bs: the LDS stages, A_STAGE and B_STAGE floats apart.
// (Offsets from one base keep the pointers visibly in LDS for the compiler;
// an array of stage pointers would turn every LDS access into a flat one.)
template <int WTM, int WTN, int BKT, int PATH, bool PRIO, int WGM = 2, int WGN = 2, int MF = 32>
__device__ __forceinline__ void gemm_tiles(const float *__restrict__ Ap, const float *__restrict__ Bp,
                                           float *__restrict__ Cp, int64_t M, int64_t N, int64_t K, int64_t lda,
                                           int64_t ldb, int64_t ldc, bool a_vec, bool b_vec, float *As,
                                           float *Bs) {
  using T = Tile<WTM, WTN, BKT, PATH == kPipeDma, WGM, WGN, MF>;
  const int tid = threadIdx.x;
  const int lane = kh::lane_id();
  const int wave = tid >> 6;
  const int wm = T::wave_m(wave), wn = T::wave_n(wave);

  const int64_t tiles_m = (M + T::BM - 1) / T::BM, tiles_n = (N + T::BN - 1) / T::BN;
  const int64_t total = tiles_m * tiles_n;
  const int64_t nslabs = (K + T::BK - 1) / T::BK;
  const int64_t gx = kh::grid_blocks_x(), gy = kh::grid_blocks_y(), gz = kh::grid_blocks_z();
  const int64_t nblocks = gx * gy * gz;
  const int64_t bid = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const bool xcd_remap = (nblocks == total) && ((total & 7) == 0);

  for (int64_t pid = bid; pid < total; pid += nblocks) {
    int64_t tm, tn;
    tile_coords(pid, tiles_m, tiles_n, xcd_remap, tm, tn);
    const int64_t m0 = tm * T::BM, n0 = tn * T::BN;

    AccOf<T> acc[WTM][WTN];
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
      for (int j = 0; j < WTN; ++j) acc[i][j] = AccOf<T>{};

    if constexpr (PATH == kPipeDma)
      k_loop_dma<WTM, WTN, T, PRIO>(acc, Ap, Bp, M, N, K, lda, ldb, m0, n0, nslabs, As, Bs, wave, wm, wn, lane);
    else if constexpr (PATH == kPipeRegs)
      k_loop_regs<WTM, WTN, T, PRIO>(acc, Ap, Bp, M, N, K, lda, ldb, m0, n0, nslabs, As, Bs, tid, wm, wn, lane);
    else if constexpr (PATH == kPipePrefetch2)
      k_loop_prefetch2<WTM, WTN, T, PRIO>(acc, Ap, Bp, M, N, K, lda, ldb, m0, n0, nslabs, As, Bs, tid, wm, wn,
                                          lane);
    else
      k_loop_generic<WTM, WTN, T>(acc, Ap, Bp, M, N, K, lda, ldb, m0, n0, nslabs, a_vec, b_vec, As, Bs, tid, wm,
                                  wn, lane);

    store_tile<WTM, WTN, T>(acc, Cp, M, N, ldc, m0, n0, wm, wn, lane);
  }
}

// ---------------------------------------------------------------------------
// Persistent pipeline (the `gemm` symbol): the workgroup loops over its
// tiles and the three-stage direct-to-LDS ring runs on across them, so the
// next tile's first two slabs are fetched during this tile's last two: no
// per-tile pipeline fill (the fill and drain are a large share of the time
// for K of a few slabs per tile).

// Asks the scheduler to interleave the fragment reads just issued with the
// MFMAs that follow them, one LDS read then one MFMA, N times (a
// chunk's fragments are WTM ds_read_b128 for A and 2 WTN ds_read2_b32 for
// B). Left to itself the compiler issued a chunk's reads as one burst
// before 32 back-to-back MFMAs. The MFMA pipe then idled whenever both
// waves of a SIMD sat in such a burst, the barrier or the slab loads at
// once. Kernel trace with variants interleaved launch by launch, same
// bits: 8192^3 7437 -> 7332 us, 4096^3 936 -> 924, 8192x8192x256 269 ->
// 265; one read per two MFMAs, or two per four, measured within 0.3% of
// that, and interleaving only one of the slab's two chunks gained half.
template <int N>
__device__ __forceinline__ void interleave_reads() {
#pragma unroll
  for (int g = 0; g < N; ++g) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
  }
}

// One slab of the persistent ring: chunk 0's MFMAs, the barrier (slab q+1
// has landed and stage fut is free), the fetch of a later slab into stage
// fut, slab q+1's first fragments, then this slab's remaining chunks. Each
// chunk's fragment reads are interleaved with the MFMAs of the chunk
// before them (interleave_reads); the wave priority is raised before the
// reads, since s_setprio bounds what the scheduler may interleave.
template <int WTM, int WTN, class T, bool PRIO, bool ALN, int WAIT = 0>
__device__ __forceinline__ void flat_step(AccOf<T> (&acc)[WTM][WTN], Frag<WTM, WTN> &f0, Frag<WTM, WTN> &f1, int &cur,
                                          const float *__restrict__ Ap, const float *__restrict__ Bp, int64_t M,
                                          int64_t N, int64_t K, int64_t lda, int64_t ldb, bool dma, int64_t dm0,
                                          int64_t dn0, int64_t dk0, bool read_next, float *As, float *Bs, int wv,
                                          int wm, int wn, int lane) {
  constexpr int C = T::BK / Mfma<T::kMF>::CK;
  constexpr int kReads = WTM + 2 * WTN;
  const int nxt = cur == 2 ? 0 : cur + 1;
  const int fut = nxt == 2 ? 0 : nxt + 1;
  const float *sA = As + cur * T::A_STAGE, *sB = Bs + cur * T::B_STAGE;
  if (PRIO) __builtin_amdgcn_s_setprio(1);
  if constexpr (C > 1) read_frag<WTM, WTN, T>(f1, sA, sB, 1, wm, wn, lane);
  mfma_frag<WTM, WTN>(acc, f0);
  if constexpr (C > 1) interleave_reads<kReads>();
  if (PRIO) __builtin_amdgcn_s_setprio(0);
  vm_barrier<WAIT>();
  if (PRIO) __builtin_amdgcn_s_setprio(1);
  float *const dA = As + fut * T::A_STAGE, *const dB = Bs + fut * T::B_STAGE;
  if constexpr (C > 1) {
    // Slab q+1's first fragments, interleaved with this slab's next MFMA
    // step; the later slab's loads, half after that step and half after
    // the one after it (each load's inline assembly is a scheduling
    // boundary, so program order places them). Against all six loads in
    // one burst before the MFMAs: 8192x8192x256 257.9 -> 253.9 us,
    // 8192^3 and 4096^3 level (7347 -> 7328, 926.0 -> 927.0 us); a 2+2+2
    // or 1+2+3 split measured slower at 8192^3 (7413-7416 us).
    constexpr int kL = T::NA + T::NB;
    if (read_next) read_frag<WTM, WTN, T>(f0, As + nxt * T::A_STAGE, Bs + nxt * T::B_STAGE, 0, wm, wn, lane);
    mfma_frag_s<WTM, WTN, 0, 1>(acc, f1);
    interleave_reads<kReads>();
    if (dma) dma_part<T, ALN, 0, kL / 2>(Ap, Bp, M, N, K, lda, ldb, dm0, dn0, dk0, dA, dB, wv, lane);
    mfma_frag_s<WTM, WTN, 1, 2>(acc, f1);
    if (dma) dma_part<T, ALN, kL / 2, kL>(Ap, Bp, M, N, K, lda, ldb, dm0, dn0, dk0, dA, dB, wv, lane);
    mfma_frag_s<WTM, WTN, 2, 4>(acc, f1);
  } else {
    if (dma) dma_slab<T, ALN>(Ap, Bp, M, N, K, lda, ldb, dm0, dn0, dk0, dA, dB, wv, lane);
    if (read_next) read_frag<WTM, WTN, T>(f0, As + nxt * T::A_STAGE, Bs + nxt * T::B_STAGE, 0, wm, wn, lane);
  }
#pragma unroll
  for (int c = 2; c < C; ++c) {
    read_frag<WTM, WTN, T>(f1, sA, sB, c, wm, wn, lane);
    mfma_frag<WTM, WTN>(acc, f1);
  }
  if (PRIO) __builtin_amdgcn_s_setprio(0);
  cur = nxt;
}

// The persistent tile loop. Slab j of the workgroup's stream sits in stage
// j % 3; slab ks of a tile fetches slab ks+2 of the same tile or, in the
// tile's last two slabs, slab 0 or 1 of the next. The tile's C stores go
// out after those fetches. Needs at least two slabs per tile (K > BK) and
// fewer than 2^31 tiles.
template <int WTM, int WTN, int BKT, bool PRIO, int WGM = 2, int WGN = 2, int MF = 32, bool ALN = false>
__device__ __forceinline__ void gemm_tiles_flat(const float *__restrict__ Ap, const float *__restrict__ Bp,
                                                float *__restrict__ Cp, int64_t M, int64_t N, int64_t K,
                                                int64_t lda, int64_t ldb, int64_t ldc, float *As, float *Bs) {
  using T = Tile<WTM, WTN, BKT, true, WGM, WGN, MF>;
  constexpr int BK = T::BK;
  constexpr int kStores = WTM * WTN * (MF == 32 ? 16 : 4);  // store_tile_buf's stores per lane
  constexpr int kStoreSlack = kStores < 62 ? kStores : 62;
  const int tid = threadIdx.x;
  const int lane = kh::lane_id();
  const int wave = tid >> 6;
  const int wm = T::wave_m(wave), wn = T::wave_n(wave);
  const int wv = __builtin_amdgcn_readfirstlane(wave);

  const int64_t tiles_m = (M + T::BM - 1) / T::BM, tiles_n = (N + T::BN - 1) / T::BN;
  const int64_t total = tiles_m * tiles_n;
  const int64_t ns = (K + BK - 1) / BK;
  const int64_t gx = kh::grid_blocks_x(), gy = kh::grid_blocks_y(), gz = kh::grid_blocks_z();
  const int64_t nblocks = gx * gy * gz;
  const int64_t bid = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  if (bid >= total) return;
  const bool xcd_remap = ((total & 7) == 0) && ((nblocks & 7) == 0);
  const int64_t mine = (total - bid + nblocks - 1) / nblocks;  // tiles of this workgroup
  // tile_coords in 32-bit arithmetic (64-bit division expands to long
  // vector-register sequences).
  const uint32_t tm32 = (uint32_t)tiles_m, tn32 = (uint32_t)tiles_n, tot32 = (uint32_t)total;
  auto coords = [&](int64_t t, int64_t &m0, int64_t &n0) {
    uint32_t pid = (uint32_t)(bid + t * nblocks);
    if (xcd_remap) pid = (pid & 7) * (tot32 >> 3) + (pid >> 3);
    const uint32_t width = kGroupM * tn32;
    const uint32_t group = pid / width;
    const uint32_t first_m = group * kGroupM;
    const uint32_t gsz = (tm32 - first_m) < (uint32_t)kGroupM ? (tm32 - first_m) : (uint32_t)kGroupM;
    const uint32_t rem = pid - group * width;
    m0 = (int64_t)(first_m + rem % gsz) * T::BM;
    n0 = (int64_t)(rem / gsz) * T::BN;
  };

  int64_t cm0, cn0;
  coords(0, cm0, cn0);
  dma_slab<T, ALN>(Ap, Bp, M, N, K, lda, ldb, cm0, cn0, 0, As, Bs, wv, lane);
  dma_slab<T, ALN>(Ap, Bp, M, N, K, lda, ldb, cm0, cn0, BK, As + T::A_STAGE, Bs + T::B_STAGE, wv, lane);
  vm_barrier<T::NA + T::NB>();
  Frag<WTM, WTN> f0, f1;
  read_frag<WTM, WTN, T>(f0, As, Bs, 0, wm, wn, lane);
  int cur = 0;
  for (int64_t t = 0; t < mine; ++t) {
    const bool has_next = t + 1 < mine;
    int64_t nm0 = 0, nn0 = 0;
    if (has_next) coords(t + 1, nm0, nn0);
    AccOf<T> acc[WTM][WTN];
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
      for (int j = 0; j < WTN; ++j) acc[i][j] = AccOf<T>{};
    {
      // Slab 0 fetches slab 2 of this tile, or slab 0 of the next (ns = 2).
      const bool same = ns > 2;
      const bool dma = same || has_next;
      const int64_t dm0 = same ? cm0 : nm0, dn0 = same ? cn0 : nn0, dk0 = same ? 2 * BK : 0;
      // The first tile's copy of this step is separate code: with one
      // shared copy the kernel measured 0.6% slower at 8192^3 and its L2
      // misses doubled (FETCH_SIZE), with the same instructions in the
      // steady-state loop.
      // In later tiles the previous tile's C stores (exactly kStores per
      // lane, issued after slab 1's loads) are still in flight. Vector
      // memory operations retire in issue order, so waiting until at most
      // min(kStores, 62) are outstanding completes the loads and lets the
      // newest stores drain behind this tile's MFMAs.
      if (t > 0)
        flat_step<WTM, WTN, T, PRIO, ALN, kStoreSlack>(acc, f0, f1, cur, Ap, Bp, M, N, K, lda, ldb, dma, dm0, dn0,
                                                       dk0, true, As, Bs, wv, wm, wn, lane);
      else
        flat_step<WTM, WTN, T, PRIO, ALN>(acc, f0, f1, cur, Ap, Bp, M, N, K, lda, ldb, dma, dm0, dn0, dk0, true, As, Bs,
                                     wv, wm, wn, lane);
    }
    for (int64_t ks = 1; ks < ns - 2; ++ks)
      flat_step<WTM, WTN, T, PRIO, ALN>(acc, f0, f1, cur, Ap, Bp, M, N, K, lda, ldb, true, cm0, cn0, (ks + 2) * BK,
                                      true, As, Bs, wv, wm, wn, lane);
    // The last two slabs (the last one only, when ns = 2) fetch the next
    // tile's slabs 0 and 1.
    for (int64_t ks = ns > 2 ? ns - 2 : 1; ks < ns; ++ks)
      flat_step<WTM, WTN, T, PRIO, ALN>(acc, f0, f1, cur, Ap, Bp, M, N, K, lda, ldb, has_next, nm0, nn0,
                                      (ks + 2 - ns) * BK, ks + 1 < ns || has_next, As, Bs, wv, wm, wn, lane);
    store_tile_buf<WTM, WTN, T>(acc, Cp, M, N, ldc, cm0, cn0, wm, wn, lane);
    cm0 = nm0;
    cn0 = nn0;
  }
}

// LDS floats a configuration needs for A and for B: the fast pipeline's
// stages (three for direct-to-LDS, two otherwise) or the generic path's one.
template <int WTM, int WTN, int BKT, int PIPE, int WGM = 2, int WGN = 2, int MF = 32>
struct LdsNeed {
  using T = Tile<WTM, WTN, BKT, PIPE == kPipeDma, WGM, WGN, MF>;
  using G = Tile<WTM, WTN, BKT, false, WGM, WGN, MF>;
  static constexpr int kStages = PIPE == kPipeDma ? 3 : 2;
  static constexpr int A = kStages * T::A_STAGE > G::A_STAGE ? kStages * T::A_STAGE : G::A_STAGE;
  static constexpr int B = kStages * T::B_STAGE > G::B_STAGE ? kStages * T::B_STAGE : G::B_STAGE;
};

// Kernel body over LDS the caller provides (LdsNeed floats each): the fast
// pipeline PIPE for aligned operands with k and n multiples of 4 and 32-bit
// tile offsets, the generic path otherwise.
template <int WTM, int WTN, int BKT, bool PRIO, int PIPE, int WGM = 2, int WGN = 2, int MF = 32>
__device__ __forceinline__ void gemm_body(const float *__restrict__ Ap, const float *__restrict__ Bp,
                                          float *__restrict__ Cp, int64_t M, int64_t N, int64_t K, int64_t lda,
                                          int64_t ldb, int64_t ldc, float *As, float *Bs) {
  using T = Tile<WTM, WTN, BKT, PIPE == kPipeDma, WGM, WGN, MF>;
  const bool a_vec = ((K & 3) == 0) && ((lda & 3) == 0) && kh::aligned16(Ap);
  const bool b_vec = ((N & 3) == 0) && ((ldb & 3) == 0) && kh::aligned16(Bp);
  // The fast loads address a tile's rows with 32-bit byte offsets.
  const bool fits32 = (int64_t)T::BM * lda * 4 < (1ll << 31) && (int64_t)T::BK * ldb * 4 < (1ll << 31);
  if (a_vec && b_vec && fits32)
    gemm_tiles<WTM, WTN, BKT, PIPE, PRIO, WGM, WGN, MF>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, a_vec, b_vec, As, Bs);
  else
    gemm_tiles<WTM, WTN, BKT, 0, PRIO, WGM, WGN, MF>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, a_vec, b_vec, As, Bs);
}

// Kernel body with its own LDS and fast pipeline PIPE.
template <int WTM, int WTN, int BKT, bool PRIO, int PIPE, int WGM = 2, int WGN = 2, int MF = 32>
__device__ __forceinline__ void gemm_entry_pipe(const float *__restrict__ Ap, const float *__restrict__ Bp,
                                                float *__restrict__ Cp, int64_t M, int64_t N, int64_t K, int64_t lda,
                                                int64_t ldb, int64_t ldc) {
  using L = LdsNeed<WTM, WTN, BKT, PIPE, WGM, WGN, MF>;
  __shared__ __attribute__((aligned(16))) float As[L::A];
  __shared__ __attribute__((aligned(16))) float Bs[L::B];
  gemm_body<WTM, WTN, BKT, PRIO, PIPE, WGM, WGN, MF>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, As, Bs);
}

// Kernel body of the persistent variant: gemm_tiles_flat when A and B are
// 16-byte aligned with k and n multiples of 4, K > BK and the tile offsets
// fit 32 bits (its tail-free form when K and N are whole slabs and tiles);
// the direct-to-LDS per-tile pipeline (or the generic path) otherwise. Same
// LDS as gemm_entry_pipe's direct-to-LDS form.
template <int WTM, int WTN, int BKT, bool PRIO, int WGM = 2, int WGN = 2, int MF = 32>
__device__ __forceinline__ void gemm_entry_flat(const float *__restrict__ Ap, const float *__restrict__ Bp,
                                                float *__restrict__ Cp, int64_t M, int64_t N, int64_t K, int64_t lda,
                                                int64_t ldb, int64_t ldc) {
  using T = Tile<WTM, WTN, BKT, true, WGM, WGN, MF>;
  using L = LdsNeed<WTM, WTN, BKT, kPipeDma, WGM, WGN, MF>;
  __shared__ __attribute__((aligned(16))) float As[L::A];
  __shared__ __attribute__((aligned(16))) float Bs[L::B];
  const bool vec = ((K & 3) == 0) && ((lda & 3) == 0) && kh::aligned16(Ap) && ((N & 3) == 0) &&
                   ((ldb & 3) == 0) && kh::aligned16(Bp);
  const bool fits32 = (int64_t)T::BM * lda * 4 < (1ll << 31) && (int64_t)T::BK * ldb * 4 < (1ll << 31) &&
                      (int64_t)T::BM * ldc * 4 < (1ll << 31);
  const int64_t tiles = ((M + T::BM - 1) / T::BM) * ((N + T::BN - 1) / T::BN);
  if (vec && fits32 && K > T::BK && tiles < (1ll << 31)) {
    // Tail-free slab loads where no slab reaches past K or N: +2-3% at
    // 8192^3, 4096^3 and 8192x8192x{256,1024} (their offsets stay in
    // registers; the general form's selects spill them around the loop).
    if (K % T::BK == 0 && N % T::BN == 0)
      gemm_tiles_flat<WTM, WTN, BKT, PRIO, WGM, WGN, MF, true>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, As, Bs);
    else
      gemm_tiles_flat<WTM, WTN, BKT, PRIO, WGM, WGN, MF, false>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, As, Bs);
  } else {
    gemm_body<WTM, WTN, BKT, PRIO, kPipeDma, WGM, WGN, MF>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc, As, Bs);
  }
}

// The same with DMA selecting the direct-to-LDS pipeline, else the
// register-staged one.
template <int WTM, int WTN, int BKT, bool PRIO, bool DMA>
__device__ __forceinline__ void gemm_entry(const float *__restrict__ Ap, const float *__restrict__ Bp,
                                           float *__restrict__ Cp, int64_t M, int64_t N, int64_t K, int64_t lda,
                                           int64_t ldb, int64_t ldc) {
  gemm_entry_pipe<WTM, WTN, BKT, PRIO, DMA ? kPipeDma : kPipeRegs>(Ap, Bp, Cp, M, N, K, lda, ldb, ldc);
}

}  // namespace khg
