// Non-causal scaled dot-product attention for gfx950 on the matrix cores:
//   O[b,h,i,:] = softmax_t(Q[b,h,i,:] . K[b,h,t,:] / sqrt(d)) V[b,h,t,:]
// fp32 throughout (v_mfma_f32_32x32x2f32), head_dim d = 64.
//
// Symbol and memref arguments follow the reference template
// (lib/dsl/kernels/attention.cpp:86-289): Q, K, V, O rank-4 [b, h, s, d],
// 44 parameters; d pinned to 64 (attention.cpp:115-120). The reference runs
// one 64-thread block per query row and recomputes q.k_t in every thread
// (attention.cpp:250-261). Here one workgroup owns 128 query rows of one
// (b, h) slice (32 per wave), streams the keys in tiles of 64 through LDS,
// and keeps the online-softmax state (running max m, running sum l) in
// registers, the same recurrence as the reference (attention.cpp:268-276):
//   m' = max(m, S);  l' = l e^{m-m'} + e^{S-m'};  acc' = acc e^{m-m'} + e^{S-m'} v.
//
// MFMA formulation (per wave, per 32-key sub-tile):
//   S^T = K Q^T        A = K rows from LDS, B = Q^T held in registers for
//                      the whole kernel (pre-scaled by log2(e)/sqrt(d), so
//                      exp becomes one v_exp_f32 of S - m).
//                      Result lane l holds query l%32 and 16 keys.
//   O^T += V^T P^T     A = V^T rows from LDS (stored transposed), B = the P
//                      registers exactly as the first product left them:
//                      MFMA k-step j of a sub-tile takes key 8(j/4)+j%4 in
//                      lane half 0 and key 8(j/4)+4+j%4 in half 1, which is
//                      where S^T put them. No register shuffles.
//   Each query lives in one lane pair (l, l^32): its max needs one cross-half
//   exchange per tile, its sum one at the end; O^T's rows are head-dim
//   elements, so the final store is four dwordx4 per lane per 32 columns.
//
// Pipelining: within one wave, tile t's softmax needs tile t's S^T, and its
// PV MFMAs need the softmax, but tile t+1's S^T needs only K. So K runs one
// tile ahead of V through the two LDS buffers, and each iteration issues
// tile t+1's S^T MFMAs alongside tile t's softmax VALU work; the exp, max
// and scaling then run while the wave's own MFMAs execute instead of only in
// the other wave's shadow (131 -> 135 TFLOP/s at b4 h16 s4096). The loop
// covers the tiles that have a successor, all full, with no branches inside
// (K/V arrive by range-checked buffer loads); the last tile, the only one
// that can be partial, is masked and finished after it.
//
// Tails: query rows >= seq are computed from zeros and not stored; key rows
// >= seq get S = -inf and V = 0. Query tiles are grid-strided in x, so any
// grid is correct, including the reference's (seq, heads, batch) x 64
// geometry (kernelh_backend.cpp:420-422). Workgroups of exactly 256 threads
// over 16-byte aligned rows of at least 64 floats take the pipelined path;
// other launches stage each tile synchronously, and rows that are not
// 16-byte aligned are read and written a float at a time. Q, K, V and O each
// use their own descriptor's strides. Descriptors that are not four
// [batch, heads, seq, 64] tensors with contiguous rows are refused: O := NaN.
#include "kh_device.h"
#include "kh_tiles.h"

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int D = 64;          // head_dim
constexpr int TK = 64;         // keys per tile
constexpr int QW = 32;         // query rows per wave
constexpr int LDK = D + 4;     // K tile in LDS: [key][d], padded rows
constexpr int LDV = TK + 4;    // V^T tile in LDS: [d][key], padded rows
constexpr int kFastThreads = 256;
constexpr float kNegBig = -1e30f;  // finite "minus infinity" seed for m


// Any workgroup size: synchronous strided staging of one tile.
__device__ __forceinline__ void stage_kv_generic(float *__restrict__ Ks, float *__restrict__ Vt,
                                                 const float *__restrict__ Kg, const float *__restrict__ Vg,
                                                 int64_t ks, int64_t vs, int64_t key0, int64_t seq, int bd) {
  for (int e = threadIdx.x; e < TK * D; e += bd) {
    const int key = e / D, d = e % D;
    const int64_t kk = key0 + key;
    Ks[key * LDK + d] = kk < seq ? Kg[kk * ks + d] : 0.0f;
    Vt[d * LDV + key] = kk < seq ? Vg[kk * vs + d] : 0.0f;
  }
}

__device__ __forceinline__ float comp(const float4 &v, int s) {
  return s == 0 ? v.x : s == 1 ? v.y : s == 2 ? v.z : v.w;
}

// S^T of one key tile for one wave (64 MFMAs).
__device__ __forceinline__ void qk_tile(v16f (&s)[2], const float4 (&q)[8], const float *__restrict__ Ks, int lane) {
  const int r = lane & 31, h = lane >> 5;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    s[kt] = v16f{};
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
      const float4 a = *reinterpret_cast<const float4 *>(Ks + (kt * 32 + r) * LDK + 8 * c + 4 * h);
#pragma unroll
      for (int st = 0; st < 4; ++st)
        s[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(comp(a, st), comp(q[c], st), s[kt], 0, 0, 0);
    }
  }
}

// Asks the scheduler to place the 16 fragment reads of the MFMA block just
// issued (qk_tile's K rows, or the PV block's V^T rows) one by one among
// its first 16 MFMAs. Left to itself it issued them as a burst ahead of the
// MFMAs, and a wave waited on LDS about once per LDS instruction. Same
// instructions, same MFMA order per accumulator, so the same bits. Kernel
// trace, variants interleaved launch by launch over rotated inputs: 1024
// keys 142.7 -> 139.5 us, 4096 keys 2029 -> 2022 (level); after the S^T
// block alone, or with the softmax's VALU work interleaved with the S^T
// block's last 48 MFMAs, the same. One read per two or four MFMAs, or
// reads issued one or two chunks ahead, measured slower (they also took
// the registers to 253-256).
__device__ __forceinline__ void interleave_reads() {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
  }
}

// Online-softmax update of one tile's S^T (into P, in place), then O^T += V^T P^T.
template <bool MASK>
__device__ __forceinline__ void softmax_pv(v16f (&o)[2], float &m, float &l, v16f (&s)[2],
                                           const float *__restrict__ Vt, int64_t key0, int64_t seq, int lane) {
  const int r = lane & 31, h = lane >> 5;
  // Mask keys past the end (only in the last, partial tile).
  if (MASK && key0 + TK > seq) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int64_t key = key0 + kt * 32 + 8 * (j >> 2) + 4 * h + (j & 3);
        if (key >= seq) s[kt][j] = -__builtin_inff();
      }
  }
  float mt = kNegBig;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int j = 0; j < 16; ++j) mt = fmaxf(mt, s[kt][j]);
  mt = fmaxf(mt, __shfl_xor(mt, 32, kh::kWave));
  const float mn = fmaxf(m, mt);
  const float alpha = kh::exp2_hw(m - mn);
  m = mn;
  float ls = 0.0f;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float p = kh::exp2_hw(s[kt][j] - mn);
      s[kt][j] = p;
      ls += p;
    }
  l = l * alpha + ls;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[dt][j] *= alpha;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const float4 v = *reinterpret_cast<const float4 *>(Vt + (dt * 32 + r) * LDV + kt * 32 + 8 * qd + 4 * h);
#pragma unroll
        for (int st = 0; st < 4; ++st)
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(comp(v, st), s[kt][4 * qd + st], o[dt], 0, 0, 0);
      }
    }
  }
}

// Fast-path K and V staging, split so K can run a tile ahead of V. Branch-free
// buffer loads over the slice's rows: rows at or past seq read 0 through
// the hardware range check.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 as_f4(u32x4 u) {
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
}
__device__ __forceinline__ void load_k(float4 (&k)[4], __amdgpu_buffer_rsrc_t rk, int64_t ks, int64_t key0, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t off = (uint32_t)(((key0 + (tid >> 4) + 16 * i) * ks + 4 * (tid & 15)) * 4);
    k[i] = as_f4(__builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
  }
}
__device__ __forceinline__ void load_v(float4 (&v)[4], __amdgpu_buffer_rsrc_t rv, int64_t vs, int64_t key0, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t off = (uint32_t)(((key0 + (tid & 63)) * vs + 4 * ((tid >> 6) + 4 * i)) * 4);
    v[i] = as_f4(__builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
  }
}
__device__ __forceinline__ void store_k(const float4 (&k)[4], float *__restrict__ Ks, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<float4 *>(Ks + ((tid >> 4) + 16 * i) * LDK + 4 * (tid & 15)) = k[i];
}
__device__ __forceinline__ void store_v(const float4 (&v)[4], float *__restrict__ Vt, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 4 * ((tid >> 6) + 4 * i), key = tid & 63;
    Vt[(d + 0) * LDV + key] = v[i].x;
    Vt[(d + 1) * LDV + key] = v[i].y;
    Vt[(d + 2) * LDV + key] = v[i].z;
    Vt[(d + 3) * LDV + key] = v[i].w;
  }
}

// One workgroup's query tiles of one (b, h) slice. VEC4: rows of Q, K, V and
// O are 16-byte aligned (float4 access, and the pipelined path for 256-thread
// workgroups); otherwise Q and O move a float at a time and tiles are staged
// synchronously. qs, ks, vs, os: row strides (floats) of Q, K, V and O.
// Ks, Vt: two LDS tile buffers each, one tile apart.
template <bool VEC4>
__device__ __forceinline__ void attention_slice(const float *__restrict__ Qg, const float *__restrict__ Kg,
                                                const float *__restrict__ Vg, float *__restrict__ Og, int64_t qs,
                                                int64_t ks, int64_t vs, int64_t os, int64_t seq, int bd,
                                                int64_t q0, int64_t qstep, float *Ks, float *Vt) {
  const int tid = threadIdx.x;
  const int lane = kh::lane_id();
  const int wave = tid / kh::kWave;
  const int nwaves = bd / kh::kWave;
  const int r = lane & 31, h = lane >> 5;
  const int64_t rows_per_block = (int64_t)QW * nwaves;
  const int64_t nqt = (seq + rows_per_block - 1) / rows_per_block;
  const int64_t ntiles = (seq + TK - 1) / TK;
  // The fast path's buffer loads address the slices with 32-bit offsets and
  // bound K by seq rows of ks floats and V by seq rows of vs floats, so every
  // row must hold its D floats.
  const int64_t widest = ks > vs ? (ks > qs ? ks : qs) : (vs > qs ? vs : qs);
  const bool fast = VEC4 && bd == kFastThreads && ks >= D && vs >= D && qs >= D &&
                    (seq + 2 * TK) * widest * 4 < (1ll << 31);
  // log2(e)/sqrt(d): S^T comes out in log2 units, so exp(S - m) = 2^(S' - m').
  const float qscale = kh::kLog2e * 0.125f;

  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(Kg), (short)0,
                                                                      (int)(seq * ks * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(Vg), (short)0,
                                                                      (int)(seq * vs * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(Qg), (short)0,
                                                                      (int)(seq * qs * 4), 0x00020000);
  for (int64_t qt = q0; qt < nqt; qt += qstep) {
    const int64_t q_row = qt * rows_per_block + (int64_t)wave * QW + r;
    float4 kr[4], vr[4];
    float4 q[8];
    v16f o[2] = {v16f{}, v16f{}};
    float m = kNegBig, l = 0.0f;

    if (fast) {
      // K runs a tile ahead of V: iteration t computes S^T of tile t+1 while
      // tile t's softmax and PV run, so one wave's VALU work overlaps its own
      // MFMAs. Buffer j % 2 of Ks holds K of tile j, of Vt V of tile j. The
      // loop covers the tiles that have a successor (all full); the last
      // tile, the only one that can be partial, is finished after it.
      v16f sa[2], sb[2];
      {
        // K0, Q, V0 and K1 go out together (one memory latency before the
        // first MFMA, not two): loads complete in issue order, so scaling Q
        // (its first use, where the compiler waits for it) after V0 and K1
        // are issued leaves those two in flight, and the barrier before
        // tile 0's S^T fences LDS only. Q moves through a range-checked
        // buffer resource (rows at or past seq read 0): loaded under
        // `if (q_row < seq)` and scaled at once, it made the compiler wait
        // for K0 and Q before V0 and K1 went out.
        load_k(kr, rk, ks, 0, tid);
        const uint32_t qoff = (uint32_t)(4 * (q_row * qs + 4 * h));
#pragma unroll
        for (int c = 0; c < 8; ++c) q[c] = as_f4(__builtin_amdgcn_raw_buffer_load_b128(rq, qoff + 32 * c, 0, 0));
        float4 k1[4];
        load_v(vr, rv, vs, 0, tid);
        load_k(k1, rk, ks, TK, tid);
#pragma unroll
        for (int c = 0; c < 8; ++c) q[c] = make_float4(q[c].x * qscale, q[c].y * qscale, q[c].z * qscale, q[c].w * qscale);
        store_k(kr, Ks, tid);
        kh::lds_barrier();
        qk_tile(sa, q, Ks, lane);
        store_v(vr, Vt, tid);
        store_k(k1, Ks + TK * LDK, tid);
      }
      __syncthreads();
      // One pipeline step: S^T of tile t+1 into sn while tile t's softmax
      // and PV consume sc. The loop is unrolled by two so sc and sn swap
      // roles instead of being copied.
      auto step = [&](int64_t t, v16f (&sc)[2], v16f (&sn)[2]) __attribute__((always_inline)) {
        const int cur = t & 1;
        load_k(kr, rk, ks, (t + 2) * TK, tid);
        load_v(vr, rv, vs, (t + 1) * TK, tid);
        qk_tile(sn, q, Ks + (cur ^ 1) * TK * LDK, lane);
        interleave_reads();
        softmax_pv<false>(o, m, l, sc, Vt + cur * D * LDV, t * TK, seq, lane);
        interleave_reads();
        store_k(kr, Ks + cur * TK * LDK, tid);
        store_v(vr, Vt + (cur ^ 1) * D * LDV, tid);
        __syncthreads();
      };
      int64_t t = 0;
      for (; t + 2 < ntiles; t += 2) {
        step(t, sa, sb);
        step(t + 1, sb, sa);
      }
      if (t + 1 < ntiles) {
        step(t, sa, sb);
        ++t;
        sa[0] = sb[0];
        sa[1] = sb[1];
      }
      // The last tile is the only one that can be partial.
      if (seq % TK == 0)
        softmax_pv<false>(o, m, l, sa, Vt + (t & 1) * D * LDV, t * TK, seq, lane);
      else
        softmax_pv<true>(o, m, l, sa, Vt + (t & 1) * D * LDV, t * TK, seq, lane);
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float4 v = make_float4(0, 0, 0, 0);
        if (q_row < seq) {
          const float *p = Qg + q_row * qs + 8 * c + 4 * h;
          v = VEC4 ? *reinterpret_cast<const float4 *>(p) : make_float4(p[0], p[1], p[2], p[3]);
        }
        q[c] = make_float4(v.x * qscale, v.y * qscale, v.z * qscale, v.w * qscale);
      }
      for (int64_t t = 0; t < ntiles; ++t) {
        stage_kv_generic(Ks, Vt, Kg, Vg, ks, vs, t * TK, seq, bd);
        __syncthreads();
        v16f sg[2];
        qk_tile(sg, q, Ks, lane);
        softmax_pv<true>(o, m, l, sg, Vt, t * TK, seq, lane);
        __syncthreads();
      }
    }

    // O = acc / l; both halves of a lane pair hold partial sums of l.
    const float lt = l + __shfl_xor(l, 32, kh::kWave);
    const float inv = 1.0f / lt;
    if (q_row < seq) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
          const float4 v = make_float4(o[dt][4 * k4] * inv, o[dt][4 * k4 + 1] * inv, o[dt][4 * k4 + 2] * inv,
                                       o[dt][4 * k4 + 3] * inv);
          float *p = Og + q_row * os + dt * 32 + 8 * k4 + 4 * h;
          if (VEC4) {
            *reinterpret_cast<float4 *>(p) = v;
          } else {
            p[0] = v.x;
            p[1] = v.y;
            p[2] = v.z;
            p[3] = v.w;
          }
        }
    }
  }
}

}  // namespace

// Registers capped for two waves per SIMD (two workgroups per CU, as LDS
// allows): one wave's softmax VALU work then overlaps the other's MFMAs.
// Uncapped, the compiler takes more than 256 registers and halves that.
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
attention(KH_MEMREF4(const float, Q), KH_MEMREF4(const float, K), KH_MEMREF4(const float, V),
          KH_MEMREF4(float, O)) {
  const float *__restrict__ Qp = KH_PTR(Q);
  const float *__restrict__ Kp = KH_PTR(K);
  const float *__restrict__ Vp = KH_PTR(V);
  float *__restrict__ Op = KH_PTR(O);
  const int64_t heads = Q_n1, seq = Q_n2;
  // The template's contract (attention.cpp:109-120 refuses other shapes):
  // four [batch, heads, seq, 64] tensors with contiguous head_dim rows.
  // Anything else is refused by filling O (as its descriptor describes it)
  // with NaN, never by computing from memory the descriptors do not cover.
  // Evaluated without short-circuit branches (& and |, not && and ||): the
  // compiler then issues every descriptor load in one round at the start
  // instead of one round per branch.
  const bool same = (K_n0 == Q_n0) & (V_n0 == Q_n0) & (O_n0 == Q_n0) & (K_n1 == heads) & (V_n1 == heads) &
                    (O_n1 == heads) & (K_n2 == seq) & (V_n2 == seq) & (O_n2 == seq);
  const bool d64 = (Q_n3 == D) & (K_n3 == D) & (V_n3 == D) & (O_n3 == D);
  const bool rows = ((Q_s3 == 1) | (Q_n3 <= 1)) & ((K_s3 == 1) | (K_n3 <= 1)) & ((V_s3 == 1) | (V_n3 <= 1)) &
                    ((O_s3 == 1) | (O_n3 <= 1));
  const int ok = same & d64 & rows;
  // The check's loads, the base pointers and the launch geometry in one round.
  const uint32_t gxy = kh::group_size_word(), bcx = kh::grid_blocks_x();
  KH_ARGS_READY(ok, Q_base, Q_off, K_base, K_off, V_base, V_off, O_base, O_off, gxy, bcx);
  if (!ok) {
    const int64_t total = O_n0 * O_n1 * O_n2 * O_n3;
    const int64_t tx = kh::threads_x_of(gxy), ty = kh::threads_y_of(gxy), tz = kh::threads_z_of(kh::group_size_z_word());
    const int64_t gy = kh::grid_blocks_y(), gz = kh::grid_blocks_z();
    const int64_t threads = tx * ty * tz;
    const int64_t flat = ((int64_t)threadIdx.z * ty + threadIdx.y) * tx + threadIdx.x;
    const int64_t block = ((int64_t)blockIdx.z * gy + blockIdx.y) * bcx + blockIdx.x;
    const int64_t step = threads * bcx * gy * gz;
    for (int64_t e = block * threads + flat; e < total; e += step) {
      int64_t r = e;
      const int64_t i3 = r % O_n3;
      r /= O_n3;
      const int64_t i2 = r % O_n2;
      r /= O_n2;
      const int64_t i1 = r % O_n1;
      const int64_t i0 = r / O_n1;
      Op[i0 * O_s0 + i1 * O_s1 + i2 * O_s2 + i3 * O_s3] = __builtin_nanf("");
    }
    return;
  }
  // Which slice and query tiles this workgroup takes: slice (blockIdx.z,
  // blockIdx.y), query tiles blockIdx.x, + gridDim.x, ... (any grid). Under
  // the launcher's grid (one workgroup per 128-row query tile of each
  // slice, slices a multiple of 8), the flat workgroup index L is remapped
  // instead so that the query tiles of a slice share an XCD: consecutive
  // workgroups go round-robin to the 8 XCDs, each with its own L2, so with
  // x the query tile a slice's tiles ran on 8 XCDs and each XCD's L2
  // fetched the slice's K and V again (HBM reads 5.7x the algorithmic K
  // and V at seq 1024). Slice = 8 (L / 8 / tiles) + L % 8, tile = (L / 8)
  // % tiles: workgroups L and L + 8 share an XCD and, mostly, a slice.
  int64_t hb = blockIdx.y, bb = blockIdx.z, q0 = blockIdx.x, qstep = bcx;
  {
    const int64_t tiles = (seq + KH_ATTN_BLOCK_Q - 1) / KH_ATTN_BLOCK_Q;
    const int64_t slices = heads * Q_n0;
    const uint32_t gy = kh::grid_blocks_y(), gz = kh::grid_blocks_z();
    if (kh::threads_x_of(gxy) == kFastThreads && (int64_t)bcx == tiles && (int64_t)gy == heads &&
        (int64_t)gz == Q_n0 && (slices & 7) == 0 && slices * tiles < (1ll << 31)) {
      const uint32_t L = (blockIdx.z * gy + blockIdx.y) * bcx + blockIdx.x;
      const uint32_t j = L >> 3, slice = (uint32_t)(j / tiles) * 8 + (L & 7);
      q0 = j % tiles;
      qstep = tiles;  // one tile per workgroup
      hb = slice % heads;
      bb = slice / heads;
    }
  }
  if (hb >= heads || bb >= Q_n0) return;
  // Row stride of the [s, d] slice is s2 (d contiguous, s3 == 1).
  const float *__restrict__ Qg = Qp + bb * Q_s0 + hb * Q_s1;
  const float *__restrict__ Kg = Kp + bb * K_s0 + hb * K_s1;
  const float *__restrict__ Vg = Vp + bb * V_s0 + hb * V_s1;
  float *__restrict__ Og = Op + bb * O_s0 + hb * O_s1;

  __shared__ __attribute__((aligned(16))) float Ks[2 * TK * LDK];
  __shared__ __attribute__((aligned(16))) float Vt[2 * D * LDV];

  // float4 access to Q, K, V and O needs 16-byte aligned rows.
  const bool vec4 = kh::aligned16(Qp) & kh::aligned16(Kp) & kh::aligned16(Vp) & kh::aligned16(Op) &
                    (((Q_s0 | Q_s1 | Q_s2 | K_s0 | K_s1 | K_s2 | V_s0 | V_s1 | V_s2 | O_s0 | O_s1 | O_s2) & 3) == 0);
  if (vec4)
    attention_slice<true>(Qg, Kg, Vg, Og, Q_s2, K_s2, V_s2, O_s2, seq, (int)kh::threads_x_of(gxy), q0, qstep, Ks, Vt);
  else
    attention_slice<false>(Qg, Kg, Vg, Og, Q_s2, K_s2, V_s2, O_s2, seq, (int)kh::threads_x_of(gxy), q0, qstep, Ks,
                           Vt);
}
