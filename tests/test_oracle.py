"""Pins the CPU oracle (oracle/oracle.c) before any GPU result is trusted.

Each oracle function is checked against something that does not share its
code: a published known answer, an independent library routine (numpy,
scipy, torch on the CPU in float64), a closed form, or an exact rational
computation on a tiny input; and each check is chosen so that a plausible
slip (dropped term, wrong sign, swapped operand, off-by-one) fails it.
The template emulators are then measured against the pinned references with
the reference's own tolerances.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle as O


# ------------------------------------------------------------------ generators

def test_mt19937_standard_known_answer():
    # C++ [rand.predef]: the 10000th invocation of a default-constructed
    # std::mt19937 (seed 5489) produces 4123659995.
    assert int(O.mt19937_raw(5489, 10000)[-1]) == 4123659995


def test_mt19937_fill_is_scaled_generator():
    raw = O.mt19937_raw(0x29C0FFEE, 1000)
    v = O.mt19937_fill(1000, 0x29C0FFEE)
    # float(uint32) rounds to 24 bits, then * 2^-32 is exact.
    assert np.array_equal(v, raw.astype(np.float32) * np.float32(2.0 ** -32))
    assert v.min() >= 0.0 and v.max() < 1.0


def test_splitmix64_known_answer():
    # Reference outputs of SplitMix64 seeded with 0 (Vigna's splitmix64.c).
    assert O.splitmix64(0, 3) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_lcg_state_sequence_matches_numerical_recipes():
    # ranqd1 (Numerical Recipes 2nd ed., sec. 7.1) from idum = 0:
    # 1013904223, 1196435762, 3519870697, 2868466484.
    seed = 0
    states = []
    for _ in range(4):
        _, seed = O.lcg_fill(1, seed)
        states.append(seed)
    assert states == [1013904223, 1196435762, 3519870697, 2868466484]
    v, _ = O.lcg_fill(100000, 0x27AB13)
    assert v.min() >= -1.0 and v.max() < 1.0
    # Values are k/32768 - 1 for k in [0, 65535]: on the 2^-15 grid.
    k = (v.astype(np.float64) + 1.0) * 32768.0
    assert np.array_equal(k, np.round(k))


def test_uniform_grid_and_range():
    u = O.uniform(1 << 16, 7, 0.0, 1.0)
    assert u.min() >= 0.0 and u.max() < 1.0
    g = u.astype(np.float64) * 2.0 ** 24
    assert np.array_equal(g, np.round(g))
    s = O.uniform(1 << 16, 7, -1.0, 1.0)
    assert np.array_equal(s.astype(np.float64), 2.0 * u.astype(np.float64) - 1.0)


def test_normal_moments():
    z = O.normal(1 << 20, 11, 0.0, 4.0).astype(np.float64)
    assert abs(z.mean()) < 0.02
    assert abs(z.std() - 4.0) < 0.02


# ------------------------------------------------------------------ vecadd

def test_vecadd_reference_exact_fill():
    n = 100000
    a, b = O.vecadd_inputs(n)
    i = np.arange(n)
    # Closed form in exact rational terms: a = (i%257)/2, b = (i%331)/4 + 1/2.
    exact = (i % 257) * 0.5 + (i % 331) * 0.25 + 0.5
    c = O.ref_vecadd(a, b)
    assert np.array_equal(c.astype(np.float64), exact)
    # Negative control premise: a - b differs on every element (b != 0).
    assert np.all(c != (a - b))


def test_vecadd_reference_is_correctly_rounded():
    rng = np.random.default_rng(1)
    a = (rng.standard_normal(1 << 16) * 10.0 ** rng.integers(-20, 20, 1 << 16)).astype(np.float32)
    b = (rng.standard_normal(1 << 16) * 10.0 ** rng.integers(-20, 20, 1 << 16)).astype(np.float32)
    # numpy's float32 add is the IEEE correctly rounded sum.
    assert np.array_equal(O.ref_vecadd(a, b), a + b)


# ------------------------------------------------------------------ softmax

def test_softmax_reference_vs_scipy():
    from scipy.special import softmax as sp_softmax
    rows, cols = 64, 1024
    x = O.normal(rows * cols, 3, 0.0, 4.0)
    y = O.ref_softmax(x, rows, cols)
    ref = sp_softmax(x.reshape(rows, cols).astype(np.float64), axis=1)
    assert np.max(np.abs(y - ref)) < 1e-13
    assert np.max(np.abs(y.sum(axis=1) - 1.0)) < 1e-12


def test_softmax_reference_closed_forms():
    # Two columns: softmax = logistic sigmoid of the difference.
    x = np.array([0.5, -1.25, 3.0, 3.0], np.float32)
    y = O.ref_softmax(x, 2, 2)
    s = 1.0 / (1.0 + np.exp(-1.75))
    assert abs(y[0, 0] - s) < 1e-15 and abs(y[0, 1] - (1 - s)) < 1e-15
    assert y[1, 0] == 0.5 and y[1, 1] == 0.5
    # Stability pattern {1000, -1000, 0, .5, -.5} (e2e_softmax_test.cpp:202-254):
    # only the +1000 entries carry weight, each 1/(#entries of 1000).
    cols = 1000
    pat = np.array([1000.0, -1000.0, 0.0, 0.5, -0.5], np.float32)
    x = np.tile(pat, cols // 5)
    y = O.ref_softmax(x, 1, cols)[0]
    assert np.all(np.isfinite(y))
    assert np.allclose(y[0::5], 1.0 / (cols // 5), rtol=0, atol=1e-15)
    assert np.max(np.delete(y, np.arange(0, cols, 5))) < 1e-300


# ------------------------------------------------------------------ layernorm

def test_layernorm_reference_vs_torch():
    import torch
    rows, cols = 32, 1024
    x = O.normal(rows * cols, 5, 0.0, 4.0)
    g = O.uniform(cols, 6, 0.5, 1.5)
    b = O.uniform(cols, 8, -0.1, 0.1)
    y = O.ref_layernorm(x, g, b, rows, cols)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x.reshape(rows, cols).astype(np.float64)), (cols,),
                                         torch.from_numpy(g.astype(np.float64)),
                                         torch.from_numpy(b.astype(np.float64)), eps=1e-5).numpy()
    assert np.max(np.abs(y - ref)) < 1e-12


def test_layernorm_reference_constant_row_and_eps0():
    cols = 256
    g, _ = O.lcg_fill(cols, 0xC0578A)
    b, _ = O.lcg_fill(cols, 0x1234)
    x = np.full(cols, 3.0, np.float32)
    y = O.ref_layernorm(x, g, b, 1, cols)[0]
    assert np.array_equal(y, b.astype(np.float64))  # var = 0 -> y = beta exactly
    y0 = O.ref_layernorm(x, g, b, 1, cols, eps=0.0)[0]
    assert np.all(np.isnan(y0))  # the negative control's NaN premise


# ------------------------------------------------------------------ scan

def test_scan_reference_exact_rational_tiny():
    x = O.mt19937_fill(300, 0x29C0FFEE)
    acc = Fraction(0)
    exact = []
    for v in x:
        acc += Fraction(float(v))
        exact.append(float(acc))  # float(Fraction) rounds correctly to fp64
    y = O.ref_scan(x)
    assert np.array_equal(y, np.array(exact).astype(np.float32))


def _f32_round_exact(q: Fraction) -> float:
    """Round a rational to the nearest fp32 (ties to even) by rational
    arithmetic alone: quantum 2^(e-23) for 2^e <= |q| < 2^(e+1), never below
    the subnormal quantum 2^-149."""
    if q == 0:
        return 0.0
    sign, q = (-1.0 if q < 0 else 1.0), abs(q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    quantum = Fraction(2) ** (max(e, -126) - 23)
    t = q / quantum
    k = t.numerator // t.denominator
    rem = t - k
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and k % 2 == 1):
        k += 1
    return sign * float(k * quantum)  # k <= 2^24: exact in fp32 and fp64


def test_scan_exact_reference_vs_rationals():
    # Wide exponents (subnormals to 2^100), both signs, cancellation, and
    # hand-made ties: 1 + 2^-24 rounds to even (1.0), 1 + 3*2^-24 up to
    # 1 + 2^-22, and 1 + 2^-24 + 2^-60 just above the tie, to 1 + 2^-23,
    # which an fp64 running sum (2^-60 lost below its ulp) rounds to 1.0.
    rng = np.random.default_rng(7)
    wide = (rng.standard_normal(1500) * np.exp2(rng.integers(-140, 100, 1500).astype(np.float64))).astype(np.float32)
    ties = np.array([1.0, 2.0 ** -24, -1.0, -(2.0 ** -24), 1.0, 3 * 2.0 ** -24, -1.0, -3 * 2.0 ** -24,
                     1.0, 2.0 ** -24, 2.0 ** -60, np.float32(1e-45), -np.float32(1e-45)], np.float32)
    for x in (wide, ties, np.concatenate([wide[:200], -wide[:200]])):
        y, a = O.ref_scan_exact(x, with_abs=True)
        acc, sabs, exact = Fraction(0), 0.0, []
        for v in x:
            acc += Fraction(float(v))
            exact.append(_f32_round_exact(acc))
        assert np.array_equal(y, np.array(exact, np.float32))
        assert np.allclose(a, np.cumsum(np.abs(x.astype(np.float64))), rtol=1e-12, atol=0)
    y = O.ref_scan_exact(ties)
    assert y[1] == 1.0 and y[5] == np.float32(1 + 2.0 ** -22) and y[10] == np.float32(1 + 2.0 ** -23)
    assert O.ref_scan(ties)[10] == 1.0  # the fp64 prefix misses it: the exact one is needed off the grid
    # On the tests' grid inputs the fp64 prefix is exact, so the two agree.
    g = O.mt19937_fill(1 << 16, 0x29C0FFEE)
    assert np.array_equal(O.ref_scan_exact(g), O.ref_scan(g))


def test_scan_exact_margin_vs_rationals():
    """The exact scan's margin (how far each exact prefix P lies from where
    its fp32 rounding r would change: min(spacing below r, spacing above
    r) / 2 - |P - r|) against exact rational arithmetic, on wide-exponent
    inputs, cancellation and hand-made ties (a tie has margin <= 0)."""
    rng = np.random.default_rng(11)
    wide = (rng.standard_normal(800) * np.exp2(rng.integers(-30, 40, 800).astype(np.float64))).astype(np.float32)
    ties = np.array([1.0, 2.0 ** -24, -1.0, -(2.0 ** -24), 3.0, 2.0 ** -22, 2.0 ** -60, -3.0], np.float32)
    for x in (wide, ties):
        y, m = O.ref_scan_exact(x, with_margin=True)
        acc = Fraction(0)
        for i, v in enumerate(x):
            acc += Fraction(float(v))
            r = np.float32(y[i])
            below = Fraction(float(r)) - Fraction(float(np.nextafter(r, np.float32(-np.inf))))
            above = Fraction(float(np.nextafter(r, np.float32(np.inf)))) - Fraction(float(r))
            want = min(below, above) / 2 - abs(acc - Fraction(float(r)))
            scale = max(abs(acc), min(below, above))
            assert abs(Fraction(float(m[i])) - want) <= scale * Fraction(1, 2 ** 50), (i, float(m[i]), float(want))
    _, m = O.ref_scan_exact(ties, with_margin=True)
    assert m[1] < 0  # 1 + 2^-24: exactly halfway to 1 + 2^-23


def test_scan_reference_vs_numpy_and_exclusive():
    x = O.uniform(1 << 20, 42, 0.0, 1.0)
    y = O.ref_scan(x)
    assert np.array_equal(y, np.cumsum(x.astype(np.float64)).astype(np.float32))
    ye = O.ref_scan(x, exclusive=True)
    assert ye[0] == 0.0
    assert np.array_equal(ye[1:], y[:-1])


# ------------------------------------------------------------------ fused_gelu

def test_gelu_reference_vs_torch_tanh_gelu():
    import torch
    x = O.normal(1 << 16, 9, 0.0, 1.0)
    y = O.ref_gelu(x)
    t = 1.5 * torch.from_numpy(x.astype(np.float64)) + 0.5
    ref = torch.nn.functional.gelu(t, approximate="tanh").numpy()
    # The template constant 0.7978845608 differs from sqrt(2/pi) by 2.9e-12.
    assert np.max(np.abs(y - ref)) < 1e-10
    # Closed forms: t = 0 (x = -1/3 is not exact; use x with t exactly 0.5).
    y1 = O.ref_gelu(np.array([0.0], np.float32))[0]
    z = 0.7978845608 * (0.5 + 0.044715 * 0.125)
    assert abs(y1 - 0.25 * (1 + np.tanh(z))) < 1e-16
    # Negative control premise: dropping tanh moves the output by > 1e-4.
    yn = O.ref_gelu(x, with_tanh=False)
    assert np.max(np.abs(yn - y)) > 1e-4


# ------------------------------------------------------------------ gemm

def test_gemm_reference_integer_exact():
    m, n, k = 96, 80, 512
    A, B = O.gemm_int_inputs(m, n, k)
    C = O.ref_gemm(A, B, m, n, k)
    exact = A.astype(np.int64) @ B.astype(np.int64)
    assert np.array_equal(C, exact.astype(np.float64))
    # Row subset agrees with the full computation.
    C2 = O.ref_gemm(A, B, m, n, k, row0=17, nrows=5)
    assert np.array_equal(C2, C[17:22])


def test_gemm_reference_vs_numpy_and_transpose_control():
    m = n = k = 64
    A = O.uniform(m * k, 1, -1.0, 1.0).reshape(m, k)
    B = O.uniform(k * n, 2, -1.0, 1.0).reshape(k, n)
    C = O.ref_gemm(A, B, m, n, k)
    assert np.max(np.abs(C - A.astype(np.float64) @ B.astype(np.float64))) < 1e-12
    Ct = O.ref_gemm(A, B, m, n, k, transpose_b=True)
    assert np.max(np.abs(Ct - A.astype(np.float64) @ B.astype(np.float64).T)) < 1e-12
    assert O.rel_frobenius(Ct, C) > 1e-2


# ------------------------------------------------------------------ attention

def test_attention_reference_vs_torch_sdpa():
    import torch
    b, h, s, d = 1, 2, 96, 64
    Q = O.normal(b * h * s * d, 1, 0.0, 1.0)
    K = O.normal(b * h * s * d, 2, 0.0, 1.0)
    V = O.normal(b * h * s * d, 3, 0.0, 1.0)
    bh = np.repeat(np.arange(b * h), s)
    qi = np.tile(np.arange(s), b * h)
    got = O.ref_attention_rows(Q, K, V, s, d, bh, qi)
    t = lambda a: torch.from_numpy(a.astype(np.float64).reshape(b, h, s, d))
    ref = torch.nn.functional.scaled_dot_product_attention(t(Q), t(K), t(V)).numpy().reshape(-1, d)
    assert np.max(np.abs(got - ref)) < 1e-12
    # Negative control premise: dropping 1/sqrt(d) changes the output.
    un = O.ref_attention_rows(Q, K, V, s, d, bh, qi, scaled=False)
    assert np.max(np.abs(un - got)) > 1e-2


def test_attention_reference_equal_keys_give_mean_of_values():
    s, d = 64, 64
    Q = O.normal(s * d, 4, 0.0, 1.0)
    K = np.tile(O.normal(d, 5, 0.0, 1.0), s)
    V = O.normal(s * d, 6, 0.0, 1.0)
    got = O.ref_attention_rows(Q, K, V, s, d, np.zeros(s, np.int64), np.arange(s))
    mean = V.reshape(s, d).astype(np.float64).mean(axis=0)
    assert np.max(np.abs(got - mean)) < 1e-13


# ------------------------------------------------------------------ emulators

@pytest.mark.parametrize("n", [1024, 65536, 1 << 20, 1000])
def test_scan_template_emulator_is_bit_exact(n):
    # The reference claims its double-float + 3-word template is bit-exact
    # against the round-to-fp32 fp64 prefix at exactly these sizes with the
    # mt19937 seed 0x29C0FFEE (e2e_scan_test.cpp:17-20, 225-256).
    x = O.mt19937_fill(n, 0x29C0FFEE)
    assert np.array_equal(O.emu_scan_template(x), O.ref_scan(x))


def test_template_emulators_meet_reference_tolerances():
    rows, cols = 64, 1024
    x, seed = O.lcg_fill(rows * cols, 0x27AB13)
    assert np.max(np.abs(O.emu_softmax(x, rows, cols) - O.ref_softmax(x, rows, cols))) <= 1e-4
    x, seed = O.lcg_fill(rows * cols, 0x2E2E8A)
    g, seed = O.lcg_fill(cols, seed)
    b, seed = O.lcg_fill(cols, seed)
    assert np.max(np.abs(O.emu_layernorm(x, g, b, rows, cols) - O.ref_layernorm(x, g, b, rows, cols))) <= 1e-4
    x, _ = O.lcg_fill(1 << 16, 0x3A5F91)
    assert np.max(np.abs(O.emu_gelu(x) - O.ref_gelu(x))) <= 1e-4
    m = n = k = 128
    A, B = O.gemm_int_inputs(m, n, k)
    assert np.array_equal(O.emu_gemm(A, B, m, n, k), O.ref_gemm(A, B, m, n, k).astype(np.float32))
    s, d = 128, 64
    Q, _ = O.lcg_fill(2 * s * d, 0x313A171B)
    K, _ = O.lcg_fill(2 * s * d, 0x51AC0D3E)
    V, _ = O.lcg_fill(2 * s * d, 0x29C0FFEE)
    bh = np.array([0, 1, 1], np.int64)
    qi = np.array([0, 5, 127], np.int64)
    ref = O.ref_attention_rows(Q, K, V, s, d, bh, qi)
    emu = O.emu_attention_rows(Q, K, V, s, d, bh, qi)
    assert O.attention_violation(emu, ref) <= 2e-3
