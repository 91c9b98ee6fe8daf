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
// Tails: query rows >= seq are computed from zeros and not stored; key rows
// >= seq get S = -inf and V = 0. Query tiles are grid-strided in x, so any
// grid is correct, including the reference's (seq, heads, batch) x 64
// geometry (kernelh_backend.cpp:420-422). Workgroups of exactly 256 threads
// double-buffer the K/V tiles; other sizes stage them synchronously.
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

struct KVRegs {
  float4 k[4];
  float4 v[4];
};

// Fast path (256 threads): thread t moves 4 float4 of K and 4 of V.
// K: key = t/16 + 16i, d4 = t%16 (16 lanes per key row, coalesced).
// V: key = t%64, d4 = t/64 + 4i (written transposed, consecutive lanes hit
// consecutive keys of one V^T row).
__device__ __forceinline__ void load_kv(KVRegs &r, const float *__restrict__ Kg, const float *__restrict__ Vg,
                                        int64_t ks, int64_t key0, int64_t seq, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t kk = key0 + (tid >> 4) + 16 * i;
    r.k[i] = kk < seq ? *reinterpret_cast<const float4 *>(Kg + kk * ks + 4 * (tid & 15)) : make_float4(0, 0, 0, 0);
    const int64_t vk = key0 + (tid & 63);
    r.v[i] = vk < seq ? *reinterpret_cast<const float4 *>(Vg + vk * ks + 4 * ((tid >> 6) + 4 * i))
                      : make_float4(0, 0, 0, 0);
  }
}

__device__ __forceinline__ void store_kv(const KVRegs &r, float *__restrict__ Ks, float *__restrict__ Vt, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    *reinterpret_cast<float4 *>(Ks + ((tid >> 4) + 16 * i) * LDK + 4 * (tid & 15)) = r.k[i];
    const int d = 4 * ((tid >> 6) + 4 * i), key = tid & 63;
    Vt[(d + 0) * LDV + key] = r.v[i].x;
    Vt[(d + 1) * LDV + key] = r.v[i].y;
    Vt[(d + 2) * LDV + key] = r.v[i].z;
    Vt[(d + 3) * LDV + key] = r.v[i].w;
  }
}

// Any workgroup size: synchronous strided staging of one tile.
__device__ __forceinline__ void stage_kv_generic(float *__restrict__ Ks, float *__restrict__ Vt,
                                                 const float *__restrict__ Kg, const float *__restrict__ Vg,
                                                 int64_t ks, int64_t key0, int64_t seq) {
  for (int e = threadIdx.x; e < TK * D; e += blockDim.x) {
    const int key = e / D, d = e % D;
    const int64_t kk = key0 + key;
    Ks[key * LDK + d] = kk < seq ? Kg[kk * ks + d] : 0.0f;
    Vt[d * LDV + key] = kk < seq ? Vg[kk * ks + d] : 0.0f;
  }
}

__device__ __forceinline__ float comp(const float4 &v, int s) {
  return s == 0 ? v.x : s == 1 ? v.y : s == 2 ? v.z : v.w;
}

// One key tile for one wave: S^T, online softmax update, O^T accumulation.
__device__ __forceinline__ void attend_tile(v16f (&o)[2], float &m, float &l, const float4 (&q)[8],
                                            const float *__restrict__ Ks, const float *__restrict__ Vt,
                                            int64_t key0, int64_t seq, int lane) {
  const int r = lane & 31, h = lane >> 5;
  v16f s[2];
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
  // Mask keys past the end (only in the last, partial tile).
  if (key0 + TK > seq) {
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
  const int64_t hb = blockIdx.y, bb = blockIdx.z;
  if (hb >= heads || bb >= Q_n0) return;
  // Row stride of the [s, d] slice is s2 (d contiguous, s3 == 1).
  const float *__restrict__ Qg = Qp + bb * Q_s0 + hb * Q_s1;
  const float *__restrict__ Kg = Kp + bb * K_s0 + hb * K_s1;
  const float *__restrict__ Vg = Vp + bb * V_s0 + hb * V_s1;
  float *__restrict__ Og = Op + bb * O_s0 + hb * O_s1;
  const int64_t qs = Q_s2, ks = K_s2, os = O_s2;

  __shared__ __attribute__((aligned(16))) float Ks[2][TK * LDK];
  __shared__ __attribute__((aligned(16))) float Vt[2][D * LDV];

  const int tid = threadIdx.x;
  const int lane = kh::lane_id();
  const int wave = tid / kh::kWave;
  const int nwaves = blockDim.x / kh::kWave;
  const int r = lane & 31, h = lane >> 5;
  const int64_t rows_per_block = (int64_t)QW * nwaves;
  const int64_t nqt = (seq + rows_per_block - 1) / rows_per_block;
  const int64_t ntiles = (seq + TK - 1) / TK;
  const bool fast = blockDim.x == kFastThreads;
  // log2(e)/sqrt(d): S^T comes out in log2 units, so exp(S - m) = 2^(S' - m').
  const float qscale = kh::kLog2e * 0.125f;

  for (int64_t qt = blockIdx.x; qt < nqt; qt += gridDim.x) {
    const int64_t q_row = qt * rows_per_block + (int64_t)wave * QW + r;
    float4 q[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float4 v = q_row < seq ? *reinterpret_cast<const float4 *>(Qg + q_row * qs + 8 * c + 4 * h)
                             : make_float4(0, 0, 0, 0);
      q[c] = make_float4(v.x * qscale, v.y * qscale, v.z * qscale, v.w * qscale);
    }
    v16f o[2] = {v16f{}, v16f{}};
    float m = kNegBig, l = 0.0f;

    if (fast) {
      KVRegs kv;
      load_kv(kv, Kg, Vg, ks, 0, seq, tid);
      store_kv(kv, Ks[0], Vt[0], tid);
      __syncthreads();
      for (int64_t t = 0; t < ntiles; ++t) {
        const int cur = t & 1;
        const bool more = t + 1 < ntiles;
        if (more) load_kv(kv, Kg, Vg, ks, (t + 1) * TK, seq, tid);
        attend_tile(o, m, l, q, Ks[cur], Vt[cur], t * TK, seq, lane);
        if (more) store_kv(kv, Ks[cur ^ 1], Vt[cur ^ 1], tid);
        __syncthreads();
      }
    } else {
      for (int64_t t = 0; t < ntiles; ++t) {
        stage_kv_generic(Ks[0], Vt[0], Kg, Vg, ks, t * TK, seq);
        __syncthreads();
        attend_tile(o, m, l, q, Ks[0], Vt[0], t * TK, seq, lane);
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
          *reinterpret_cast<float4 *>(Og + q_row * os + dt * 32 + 8 * k4 + 4 * h) = v;
        }
    }
  }
}
