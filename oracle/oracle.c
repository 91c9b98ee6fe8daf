/*
 * kernel.h seven-template ORACLE - test infrastructure, not product code.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker (or, for cpu_baseline, as the timed
 * CPU restatement). The GPU product path never links or calls it.
 *
 * Contents
 *   1. Input generators, bit-for-bit the reference's recipes:
 *        - the LCG fill of the e2e tests  (test/unit/e2e_softmax_test.cpp:67-74,
 *          same recipe in e2e_layernorm_test.cpp:57-64,
 *          e2e_fused_gelu_test.cpp:79-86, e2e_attention_test.cpp:71-79)
 *        - std::mt19937 * 2^-32 fill     (test/unit/e2e_scan_test.cpp:63-68)
 *        - exact vecadd fill              (test/unit/e2e_vecadd_test.cpp:40-46)
 *        - exact integer GEMM fill        (test/unit/e2e_gemm_test.cpp:70-75)
 *      plus SplitMix64 (Steele, Lea & Flood 2014) uniform / Box-Muller normal
 *      generators for the benchmark configurations.
 *   2. fp64 references restated from the reference's e2e tests (the oracle
 *      the reference itself checks its device output against).
 *   3. Emulators: fp32 restatements of each kernel template's op order
 *      (lib/dsl/kernels/<name>.cpp), used to show how far the template's own
 *      arithmetic sits from the fp64 reference.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp). FP contraction
 * is off so every emulator op rounds exactly like the template's fp32 op.
 *
 * Pinning status of every function is documented in the test suite
 * (tests/test_oracle.py); a function without an independent check there is
 * marked "parity unpinned" in its comment below.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define KHO_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* threads                                                                   */
/* ------------------------------------------------------------------------ */

static int g_threads = 1;

KHO_API void kho_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
KHO_API int kho_get_threads(void) { return g_threads; }
KHO_API int kho_openmp_enabled(void) {
#ifdef _OPENMP
  return 1;
#else
  return 0;
#endif
}

/* ------------------------------------------------------------------------ */
/* 1. generators                                                             */
/* ------------------------------------------------------------------------ */

/* LCG fill in [-1, 1): seed = seed*1664525 + 1013904223;
 * x = (float)((int32)(seed >> 8) & 0xffff) / 32768 - 1.
 * Follows test/unit/e2e_softmax_test.cpp:67-74 exactly, including the
 * float (not double) division and subtraction. The seed is carried through
 * so consecutive fills continue one stream (e2e_layernorm_test.cpp:122-125). */
KHO_API void kho_lcg_fill(float *v, size_t n, uint32_t *seed) {
  uint32_t s = *seed;
  for (size_t i = 0; i < n; ++i) {
    s = s * 1664525u + 1013904223u;
    const float q = (float)((int32_t)(s >> 8) & 0xffff);
    v[i] = q / 32768.0f - 1.0f;
  }
  *seed = s;
}

/* MT19937 (Matsumoto & Nishimura 1998), the generator std::mt19937 names:
 * w=32, n=624, m=397, r=31, a=0x9908b0df, u=11, d=0xffffffff, s=7,
 * b=0x9d2c5680, t=15, c=0xefc60000, l=18, f=1812433253. */
typedef struct {
  uint32_t mt[624];
  int idx;
} kho_mt;

static void mt_seed(kho_mt *g, uint32_t seed) {
  g->mt[0] = seed;
  for (int i = 1; i < 624; ++i) {
    g->mt[i] = 1812433253u * (g->mt[i - 1] ^ (g->mt[i - 1] >> 30)) + (uint32_t)i;
  }
  g->idx = 624;
}

static uint32_t mt_next(kho_mt *g) {
  if (g->idx >= 624) {
    for (int i = 0; i < 624; ++i) {
      const uint32_t y = (g->mt[i] & 0x80000000u) | (g->mt[(i + 1) % 624] & 0x7fffffffu);
      uint32_t v = g->mt[(i + 397) % 624] ^ (y >> 1);
      if (y & 1u) v ^= 0x9908b0dfu;
      g->mt[i] = v;
    }
    g->idx = 0;
  }
  uint32_t y = g->mt[g->idx++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

/* Raw MT19937 outputs (used to pin the generator against the C++ standard's
 * required value: the 10000th output for seed 5489 is 4123659995). */
KHO_API void kho_mt19937_raw(uint32_t seed, uint32_t *out, size_t n) {
  kho_mt g;
  mt_seed(&g, seed);
  for (size_t i = 0; i < n; ++i) out[i] = mt_next(&g);
}

/* Scan input fill: x = (float)rng() * (1.0f / 4294967296.0f)
 * (test/unit/e2e_scan_test.cpp:63-68): the uint32 -> float conversion rounds
 * to nearest, then the product is an exact power-of-two scale. */
KHO_API void kho_mt19937_fill(float *v, size_t n, uint32_t seed) {
  kho_mt g;
  mt_seed(&g, seed);
  for (size_t i = 0; i < n; ++i) {
    v[i] = (float)mt_next(&g) * (1.0f / 4294967296.0f);
  }
}

/* SplitMix64 (Steele, Lea & Flood, OOPSLA 2014). */
KHO_API uint64_t kho_splitmix64_next(uint64_t *state) {
  uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

/* Uniform on the 2^-24 grid: u = (r >> 40) * 2^-24 in [0, 1); the value is
 * lo + (hi - lo) * u evaluated in fp64, then rounded to fp32. For [0,1) and
 * [-1,1) (2u-1) the fp32 value is exact, so every such input is a multiple
 * of 2^-24 and fp64 prefix sums of up to 2^29 of them are exact. */
KHO_API void kho_fill_uniform(float *v, size_t n, uint64_t seed, double lo, double hi) {
  uint64_t st = seed;
  for (size_t i = 0; i < n; ++i) {
    const double u = (double)(kho_splitmix64_next(&st) >> 40) * (1.0 / 16777216.0);
    v[i] = (float)(lo + (hi - lo) * u);
  }
}

/* Normal(mean, std^2) by fp64 Box-Muller, then rounded to fp32. Each
 * element consumes two SplitMix64 outputs: u1 in (0,1] (53-bit), u2 in
 * [0,1); z = sqrt(-2 ln u1) cos(2 pi u2). */
KHO_API void kho_fill_normal(float *v, size_t n, uint64_t seed, double mean, double sd) {
  uint64_t st = seed;
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; ++i) {
    const double u1 = (double)((kho_splitmix64_next(&st) >> 11) + 1) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(kho_splitmix64_next(&st) >> 11) * (1.0 / 9007199254740992.0);
    const double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    v[i] = (float)(mean + sd * z);
  }
}

/* Exact-in-fp32 vecadd inputs (test/unit/e2e_vecadd_test.cpp:40-46). */
KHO_API void kho_fill_vecadd(float *a, float *b, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    a[i] = (float)(i % 257) * 0.5f;
    b[i] = (float)(i % 331) * 0.25f + 0.5f;
  }
}

/* Exact integer GEMM inputs in [0, 64) (test/unit/e2e_gemm_test.cpp:70-75):
 * A[i,k] = (i*131 + k*17 + 7) & 63, B[k,j] = (k*97 + j*41 + 3) & 63. */
KHO_API void kho_fill_gemm_int(float *A, float *B, long m, long n, long k) {
  for (long i = 0; i < m; ++i)
    for (long kk = 0; kk < k; ++kk) A[i * k + kk] = (float)((i * 131 + kk * 17 + 7) & 63);
  for (long kk = 0; kk < k; ++kk)
    for (long j = 0; j < n; ++j) B[kk * n + j] = (float)((kk * 97 + j * 41 + 3) & 63);
}

/* ------------------------------------------------------------------------ */
/* 2. fp64 references                                                        */
/* ------------------------------------------------------------------------ */

/* vecadd: fp64 sum rounded to fp32. IEEE fp32 addition is correctly rounded
 * and fp64 holds any sum of two fp32 values exactly when their exponents are
 * within 29 of each other, and rounds innocuously otherwise (53 >= 2*24+2),
 * so this equals the correctly rounded fp32 sum for all finite inputs. */
KHO_API void kho_ref_vecadd(const float *a, const float *b, float *c, size_t n) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (size_t i = 0; i < n; ++i) c[i] = (float)((double)a[i] + (double)b[i]);
}

/* softmax_reference_row (test/unit/e2e_softmax_test.cpp:78-91): true max,
 * then exp(x - max) / sum, all in fp64. Rows [row0, row0 + nrows). */
KHO_API void kho_ref_softmax(const float *x, double *y, long cols, long row0, long nrows) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (long r = row0; r < row0 + nrows; ++r) {
    const float *xr = x + (size_t)r * (size_t)cols;
    double *yr = y + (size_t)(r - row0) * (size_t)cols;
    double m = (double)xr[0];
    for (long c = 1; c < cols; ++c) m = fmax(m, (double)xr[c]);
    double s = 0.0;
    for (long c = 0; c < cols; ++c) s += exp((double)xr[c] - m);
    for (long c = 0; c < cols; ++c) yr[c] = exp((double)xr[c] - m) / s;
  }
}

/* reference_row (test/unit/e2e_layernorm_test.cpp:68-89): two-pass mean and
 * variance in fp64, inv = 1/sqrt(var + eps), y = (x-mean)*inv*gamma + beta. */
KHO_API void kho_ref_layernorm(const float *x, const float *gamma, const float *beta, double eps,
                               double *y, long cols, long row0, long nrows) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (long r = row0; r < row0 + nrows; ++r) {
    const float *xr = x + (size_t)r * (size_t)cols;
    double *yr = y + (size_t)(r - row0) * (size_t)cols;
    double mean = 0.0;
    for (long c = 0; c < cols; ++c) mean += (double)xr[c];
    mean /= (double)cols;
    double var = 0.0;
    for (long c = 0; c < cols; ++c) {
      const double d = (double)xr[c] - mean;
      var += d * d;
    }
    var /= (double)cols;
    const double inv = 1.0 / sqrt(var + eps);
    for (long c = 0; c < cols; ++c)
      yr[c] = ((double)xr[c] - mean) * inv * (double)gamma[c] + (double)beta[c];
  }
}

/* Round-to-fp32 fp64 prefix (test/unit/e2e_scan_test.cpp:159-173):
 * inclusive by default, exclusive for the negative control. The fp64
 * accumulation is exact whenever all inputs share a 2^-e grid and the
 * total needs <= 53 bits (true for every configuration the tests use). */
KHO_API void kho_ref_scan(const float *x, float *y, size_t n, int exclusive) {
  double acc = 0.0;
  for (size_t i = 0; i < n; ++i) {
    const double xv = (double)x[i];
    const double pref = exclusive ? acc : acc + xv;
    acc += xv;
    y[i] = (float)pref;
  }
}

/* Correctly rounded (round-to-nearest-even) fp32 inclusive prefix of any
 * finite fp32 inputs: the exact value the fp64 reference above approximates
 * (e2e_scan_test.cpp:159-173) and the template's double-float + 3-word
 * expansion aims for (scan.cpp:25-38). Every finite fp32 is an integer
 * multiple of 2^-149, so the running sum is kept exactly as a 320-bit
 * two's-complement integer in units of 2^-149 (a long accumulator: 277 bits
 * span the fp32 range, the rest hold the carries of up to 2^40 terms), and
 * each prefix is rounded from it once. `acc_abs` (optional) receives the
 * fp64 running sum of |x|, which error bounds for inexact summation use.
 * Pinned against Python's exact rational arithmetic (tests/test_oracle.py). */
#define KHO_LIMBS 5
static void acc_add(uint64_t *a, const uint64_t *b) {
  unsigned __int128 c = 0;
  for (int i = 0; i < KHO_LIMBS; ++i) {
    c += (unsigned __int128)a[i] + b[i];
    a[i] = (uint64_t)c;
    c >>= 64;
  }
}
static void acc_neg(uint64_t *a) {
  unsigned __int128 c = 1;
  for (int i = 0; i < KHO_LIMBS; ++i) {
    c += (uint64_t)~a[i];
    a[i] = (uint64_t)c;
    c >>= 64;
  }
}
static float acc_round_f32(const uint64_t *acc) {
  uint64_t m[KHO_LIMBS];
  memcpy(m, acc, sizeof m);
  const int neg = (int)(m[KHO_LIMBS - 1] >> 63);
  if (neg) acc_neg(m);
  int top = -1;  /* index of the highest set bit of |acc| */
  for (int i = KHO_LIMBS - 1; i >= 0 && top < 0; --i)
    if (m[i]) top = 64 * i + 63 - __builtin_clzll(m[i]);
  if (top < 0) return 0.0f;
  float r;
  if (top <= 23) {
    /* below 2^24 units of 2^-149: subnormal or the smallest normals, exact */
    r = ldexpf((float)m[0], -149);
  } else {
    /* keep 24 bits [top-23, top]; round the rest to nearest, ties to even */
    const int lo = top - 23;
    uint64_t keep = 0;
    for (int b = 0; b < 24; ++b) {
      const int bit = lo + b;
      keep |= ((m[bit >> 6] >> (bit & 63)) & 1ull) << b;
    }
    const int half = lo - 1;
    const int hbit = (int)((m[half >> 6] >> (half & 63)) & 1ull);
    int sticky = 0;
    for (int bit = 0; bit < half && !sticky; ++bit) sticky = (int)((m[bit >> 6] >> (bit & 63)) & 1ull);
    if (hbit && (sticky || (keep & 1ull))) keep += 1;
    r = ldexpf((float)keep, lo - 149);  /* keep <= 2^24: exact; overflow gives inf */
  }
  return neg ? -r : r;
}
/* The long accumulator's value as a double (rounded once, to nearest). */
static double acc_to_double(const uint64_t *acc) {
  uint64_t m[KHO_LIMBS];
  memcpy(m, acc, sizeof m);
  const int neg = (int)(m[KHO_LIMBS - 1] >> 63);
  if (neg) acc_neg(m);
  /* sum the limbs from the top: the leading ~2 limbs carry the value; the
     rounding of this sum is far below what the callers resolve */
  double v = 0.0;
  for (int i = KHO_LIMBS - 1; i >= 0; --i) v += ldexp((double)m[i], 64 * i - 149);
  return neg ? -v : v;
}

/* x as a long-accumulator integer in units of 2^-149 (x finite). */
static void acc_from_float(float x, uint64_t *t) {
  uint32_t bits;
  memcpy(&bits, &x, 4);
  const uint32_t ebits = (bits >> 23) & 0xffu;
  uint64_t mant = bits & 0x7fffffu;
  int shift = 0; /* x = mant * 2^(shift - 149) */
  if (ebits != 0) {
    mant |= 0x800000u;
    shift = (int)ebits - 1;
  }
  memset(t, 0, sizeof(uint64_t) * KHO_LIMBS);
  const int limb = shift >> 6, off = shift & 63;
  t[limb] = mant << off;
  if (off > 40 && limb + 1 < KHO_LIMBS) t[limb + 1] = mant >> (64 - off);
  if (bits >> 31) acc_neg(t);
}

/* `margin` (optional): for each prefix, how far the exact value P lies from
 * the nearest boundary where its fp32 rounding r would change,
 * min(spacing below r, spacing above r) / 2 - |P - r|, in fp64 (relative
 * error ~2^-52 of |P|). An approximation S of P with |S - P| < margin rounds
 * to r too. */
KHO_API void kho_ref_scan_exact(const float *x, float *y, size_t n, double *acc_abs, double *margin) {
  uint64_t acc[KHO_LIMBS] = {0};
  double sabs = 0.0;
  for (size_t i = 0; i < n; ++i) {
    uint64_t t[KHO_LIMBS];
    acc_from_float(x[i], t);
    acc_add(acc, t);
    y[i] = acc_round_f32(acc);
    if (acc_abs) {
      sabs += fabs((double)x[i]);
      acc_abs[i] = sabs;
    }
    if (margin) {
      /* residual P - r, exactly in the accumulator, then as a double */
      uint64_t res[KHO_LIMBS], r[KHO_LIMBS];
      memcpy(res, acc, sizeof res);
      acc_from_float(y[i], r);
      acc_neg(r);
      acc_add(res, r);
      const double below = (double)y[i] - (double)nextafterf(y[i], -INFINITY);
      const double above = (double)nextafterf(y[i], INFINITY) - (double)y[i];
      margin[i] = 0.5 * (below < above ? below : above) - fabs(acc_to_double(res));
    }
  }
}

/* gelu_reference (test/unit/e2e_fused_gelu_test.cpp:59-70): t = 1.5x + 0.5,
 * 0.5 t (1 + tanh(0.7978845608 (t + 0.044715 t^3))), fp64, with the
 * template's constants. with_tanh = 0 gives the negative control's
 * tanh(x) -> x reference (e2e_fused_gelu_test.cpp:72-76). */
KHO_API void kho_ref_gelu(const float *x, double *y, size_t n, int with_tanh) {
  const double kA = 1.5, kB = 0.5, kC = 0.7978845608, kD = 0.044715;
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (size_t i = 0; i < n; ++i) {
    const double t = kA * (double)x[i] + kB;
    const double z = kC * (t + kD * t * t * t);
    y[i] = 0.5 * t * (1.0 + (with_tanh ? tanh(z) : z));
  }
}

/* fp64 GEMM reference for rows [row0, row0 + nrows) as per-row rank-1
 * updates (test/unit/e2e_gemm_test.cpp:92-110). Output kept in fp64; the
 * reference casts to fp32 before its Frobenius check, the caller may too.
 * transpose_b = 1 computes A*B^T (the negative control, B read as [n,k]
 * with n == k). */
KHO_API void kho_ref_gemm(const float *A, const float *B, double *C, long m, long n, long k,
                          long row0, long nrows, int transpose_b) {
  (void)m;
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (long i = row0; i < row0 + nrows; ++i) {
    double *acc = C + (size_t)(i - row0) * (size_t)n;
    for (long j = 0; j < n; ++j) acc[j] = 0.0;
    for (long kk = 0; kk < k; ++kk) {
      const double av = (double)A[(size_t)i * (size_t)k + (size_t)kk];
      if (!transpose_b) {
        const float *brow = B + (size_t)kk * (size_t)n;
        for (long j = 0; j < n; ++j) acc[j] += av * (double)brow[j];
      } else {
        for (long j = 0; j < n; ++j) acc[j] += av * (double)B[(size_t)j * (size_t)k + (size_t)kk];
      }
    }
  }
}

/* attention_reference_row (test/unit/e2e_attention_test.cpp:87-122) for a
 * list of query rows. Q/K/V are [batch*heads, seq, d] contiguous; row r of
 * the list is (slice = bh[r], query = qi[r]). scaled = 0 drops the 1/sqrt(d)
 * (the negative control). Output O[r, 0..d). */
KHO_API void kho_ref_attention_rows(const float *Q, const float *K, const float *V, double *O,
                                    long seq, long d, int scaled, const int64_t *bh,
                                    const int64_t *qi, long count) {
  const double scale = scaled ? 1.0 / sqrt((double)d) : 1.0;
#pragma omp parallel num_threads(g_threads)
  {
    double *s = (double *)malloc(sizeof(double) * (size_t)seq);
#pragma omp for schedule(static)
    for (long r = 0; r < count; ++r) {
      const size_t base = (size_t)bh[r] * (size_t)seq * (size_t)d;
      const float *q = Q + base + (size_t)qi[r] * (size_t)d;
      const float *Km = K + base;
      const float *Vm = V + base;
      double m = -INFINITY;
      for (long t = 0; t < seq; ++t) {
        double dot = 0.0;
        for (long j = 0; j < d; ++j) dot += (double)q[j] * (double)Km[(size_t)t * d + j];
        s[t] = dot * scale;
        m = fmax(m, s[t]);
      }
      double l = 0.0;
      for (long t = 0; t < seq; ++t) {
        s[t] = exp(s[t] - m);
        l += s[t];
      }
      double *o = O + (size_t)r * (size_t)d;
      for (long j = 0; j < d; ++j) {
        double acc = 0.0;
        for (long t = 0; t < seq; ++t) acc += s[t] / l * (double)Vm[(size_t)t * d + j];
        o[j] = acc;
      }
    }
    free(s);
  }
}

/* ------------------------------------------------------------------------ */
/* 3. template emulators (fp32 op order of lib/dsl/kernels/<name>.cpp)         */
/* ------------------------------------------------------------------------ */

/* softmax template (lib/dsl/kernels/softmax.cpp:121-161): seed m = x[0],
 * s = 0; for every column m' = max(m,x), s = s*exp(m-m') + exp(x-m');
 * then y = exp(x - m) / s. Host expf stands in for the device exp (ocml):
 * parity of that last ulp is unpinned (the device library cannot run here). */
KHO_API void kho_emu_softmax(const float *x, float *y, long rows, long cols) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (long r = 0; r < rows; ++r) {
    const float *xr = x + (size_t)r * (size_t)cols;
    float *yr = y + (size_t)r * (size_t)cols;
    float m = xr[0], s = 0.0f;
    for (long c = 0; c < cols; ++c) {
      const float mn = fmaxf(m, xr[c]);
      s = s * expf(m - mn) + expf(xr[c] - mn);
      m = mn;
    }
    for (long c = 0; c < cols; ++c) yr[c] = expf(xr[c] - m) / s;
  }
}

/* layernorm template (lib/dsl/kernels/layernorm.cpp:106-152): serial fp32
 * sum / cols, serial sum of squared deviations / cols, rsqrt(var + 1e-5f),
 * y = ((x - mean) * inv) * gamma + beta. Host 1/sqrtf stands in for
 * ocml rsqrt (last-ulp parity unpinned). */
KHO_API void kho_emu_layernorm(const float *x, const float *gamma, const float *beta, float *y,
                               long rows, long cols) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (long r = 0; r < rows; ++r) {
    const float *xr = x + (size_t)r * (size_t)cols;
    float *yr = y + (size_t)r * (size_t)cols;
    float s1 = 0.0f;
    for (long c = 0; c < cols; ++c) s1 += xr[c];
    const float mean = s1 / (float)cols;
    float s2 = 0.0f;
    for (long c = 0; c < cols; ++c) {
      const float d = xr[c] - mean;
      s2 += d * d;
    }
    const float var = s2 / (float)cols;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
    for (long c = 0; c < cols; ++c) yr[c] = ((xr[c] - mean) * inv) * gamma[c] + beta[c];
  }
}

/* fused_gelu template after fusion (lib/dsl/kernels/fused_gelu.cpp:137-156):
 * t = fmaf(1.5, x, 0.5); t3 = (t*t)*t; z = 0.7978845608f * (t + 0.044715f*t3);
 * out = (0.5f*t) * (tanhf(z) + 1). Host tanhf stands in for ocml tanh. */
KHO_API void kho_emu_gelu(const float *x, float *y, size_t n) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (size_t i = 0; i < n; ++i) {
    const float t = fmaf(1.5f, x[i], 0.5f);
    const float t3 = (t * t) * t;
    const float z = 0.7978845608f * (t + 0.044715f * t3);
    y[i] = (0.5f * t) * (tanhf(z) + 1.0f);
  }
}

/* ---- scan template: double-float Blelloch + 3-word expansion totals ---- */

static inline void two_sum(float a, float b, float *s, float *e) {
  const float ss = a + b;
  const float bb = ss - a;
  *e = (a - (ss - bb)) + (b - bb);
  *s = ss;
}

/* dfAdd (lib/dsl/kernels/scan.cpp:113-120) */
static inline void df_add(float h1, float l1, float h2, float l2, float *hh, float *ll) {
  float s, se;
  two_sum(h1, h2, &s, &se);
  const float e2 = (se + l1) + l2;
  const float h = s + e2;
  *ll = e2 - (h - s);
  *hh = h;
}

/* dfAdd1 (scan.cpp:123-129) */
static inline void df_add1(float h, float l, float v, float *hh, float *ll) {
  float s, se;
  two_sum(h, v, &s, &se);
  const float e2 = se + l;
  const float hx = s + e2;
  *ll = e2 - (hx - s);
  *hh = hx;
}

/* grow3 (scan.cpp:134-142) */
static inline void grow3(float *e0, float *e1, float *e2, float v) {
  float a0, q, b1, q2, c2, q3;
  two_sum(*e0, v, &a0, &q);
  two_sum(*e1, q, &b1, &q2);
  two_sum(*e2, q2, &c2, &q3);
  (void)q3;
  *e0 = a0;
  *e1 = b1;
  *e2 = c2;
}

/* finalRound (scan.cpp:149-156) */
static inline float final_round(float o0, float o1, float o2, float segH, float segL) {
  float r1h, r1l, rh, rl, s, se;
  df_add(segH, segL, o1, 0.0f, &r1h, &r1l);
  df_add(r1h, r1l, o2, 0.0f, &rh, &rl);
  two_sum(o0, rh, &s, &se);
  const float e = se + rl;
  return s + e;
}

/* Both template passes (scan.cpp:163-341 and 350-453) restated serially:
 * per 256-element block a double-float Blelloch up/down sweep (padded with
 * x[n-1]), inclusive = exclusive + original, then the exact 3-word prefix of
 * the block totals and the correctly rounded combine. */
KHO_API void kho_emu_scan_template(const float *x, float *y, size_t n) {
  const size_t W = 256;
  const size_t T = (n + W - 1) / W;
  float *thi = (float *)malloc(sizeof(float) * T);
  float *tlo = (float *)malloc(sizeof(float) * T);
  float *ylo = (float *)malloc(sizeof(float) * n);
  float hi[256], lo[256], orig[256];
  for (size_t b = 0; b < T; ++b) {
    const size_t start = b * W;
    for (size_t t = 0; t < W; ++t) {
      const size_t g = start + t < n ? start + t : n - 1;
      hi[t] = x[g];
      lo[t] = 0.0f;
      orig[t] = x[g];
    }
    for (size_t stride = 2, half = 1; stride <= W; stride *= 2, half *= 2) {
      for (size_t t = 0; t < W / stride; ++t) {
        const size_t iA = t * stride + stride - 1, iB = t * stride + half - 1;
        df_add(hi[iA], lo[iA], hi[iB], lo[iB], &hi[iA], &lo[iA]);
      }
    }
    hi[W - 1] = 0.0f;
    lo[W - 1] = 0.0f;
    for (size_t stride = W, half = W / 2; stride >= 2; stride /= 2, half /= 2) {
      for (size_t t = 0; t < W / stride; ++t) {
        const size_t iA = t * stride + half - 1, iB = t * stride + stride - 1;
        const float tvH = hi[iA], tvL = lo[iA];
        const float bh = hi[iB], bl = lo[iB];
        hi[iA] = bh;
        lo[iA] = bl;
        df_add(bh, bl, tvH, tvL, &hi[iB], &lo[iB]);
      }
    }
    const size_t k = (n - start) < W ? (n - start) : W;
    for (size_t w = 0; w < k; ++w) df_add1(hi[w], lo[w], orig[w], &y[start + w], &ylo[start + w]);
    df_add1(hi[W - 1], lo[W - 1], orig[W - 1], &thi[b], &tlo[b]);
  }
  float e0 = 0.0f, e1 = 0.0f, e2 = 0.0f;
  for (size_t b = 0; b < T; ++b) {
    const float o0 = e0, o1 = e1, o2 = e2;
    grow3(&e0, &e1, &e2, thi[b]);
    grow3(&e0, &e1, &e2, tlo[b]);
    const size_t start = b * W;
    const size_t k = (n - start) < W ? (n - start) : W;
    for (size_t i = 0; i < k; ++i) y[start + i] = final_round(o0, o1, o2, y[start + i], ylo[start + i]);
  }
  free(thi);
  free(tlo);
  free(ylo);
}

/* gemm template (lib/dsl/kernels/gemm.cpp:265-296): acc = 0, then
 * acc = fmaf(a, b, acc) over k in order. Rows [row0, row0+nrows). */
KHO_API void kho_emu_gemm(const float *A, const float *B, float *C, long n, long k, long row0,
                          long nrows) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (long i = row0; i < row0 + nrows; ++i) {
    for (long j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (long kk = 0; kk < k; ++kk)
        acc = fmaf(A[(size_t)i * k + kk], B[(size_t)kk * n + j], acc);
      C[(size_t)(i - row0) * n + j] = acc;
    }
  }
}

/* attention template (lib/dsl/kernels/attention.cpp:196-287) for a list of
 * query rows: m = -1e30, l = 0, acc = 0; per key t, S = (sum_d q*k in order,
 * separate mul and add) * (1/sqrt(d) as fp32); m' = max(m,S);
 * scale = exp(m - m'); l = l*scale + exp(S-m'); acc = acc*scale + p*v;
 * O = acc / l. Host expf stands in for ocml exp. */
KHO_API void kho_emu_attention_rows(const float *Q, const float *K, const float *V, float *O,
                                    long seq, long d, const int64_t *bh, const int64_t *qi,
                                    long count) {
  const float inv_sqrt_d = (float)(1.0 / sqrt((double)d));
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (long r = 0; r < count; ++r) {
    const size_t base = (size_t)bh[r] * (size_t)seq * (size_t)d;
    const float *q = Q + base + (size_t)qi[r] * (size_t)d;
    for (long j = 0; j < d; ++j) {
      float m = -1e30f, l = 0.0f, acc = 0.0f;
      for (long t = 0; t < seq; ++t) {
        float dot = 0.0f;
        for (long e = 0; e < d; ++e) dot = dot + q[e] * K[base + (size_t)t * d + e];
        const float sv = dot * inv_sqrt_d;
        const float mn = fmaxf(m, sv);
        const float sc = expf(m - mn);
        const float p = expf(sv - mn);
        l = l * sc + p;
        acc = acc * sc + p * V[base + (size_t)t * d + j];
        m = mn;
      }
      O[(size_t)r * d + j] = acc / l;
    }
  }
}
