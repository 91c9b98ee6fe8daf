"""vecadd and fused_gelu on the GPU against the pinned oracle.

vecadd: bit-exact against the fp64 sum rounded to fp32 (the reference checks
max abs <= 1e-6 on exact inputs, e2e_vecadd_test.cpp:153-154; the exact
fill makes that 0.0). fused_gelu: max abs <= 1e-4 against the fp64
gelu_reference (e2e_fused_gelu_test.cpp:63, 293). Both include the
reference's sizes, ragged tails, unaligned descriptors, the reference's
negative controls (a-b; gelu without tanh) and the BASELINE sizes.
"""
import numpy as np
import pytest

import kernelh as kh
import oracle as O
from khtest import down, empty, say, up

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1024, 65536, 1 << 20, 1, 3, 1000, 4097, 1 << 24])
def test_vecadd_bit_exact_reference_fill(dev, n):
    a, b = O.vecadd_inputs(n)
    da, db, dc = up(a), up(b), empty(n)
    say(f"vecadd exact-fill n={n}")
    kh.vecadd(da, db, dc, n)
    got = down(dc, n)
    assert np.array_equal(got, O.ref_vecadd(a, b))
    # Negative control (e2e_vecadd_test.cpp:162-236): a - b must not match.
    assert not np.any(got == a - b)


def test_vecadd_bit_exact_bench_inputs(dev):
    n = 1 << 24  # BASELINE config: a, b ~ U[-1, 1] on the 2^-24 grid
    a = O.uniform(n, 0x5EED0001, -1.0, 1.0)
    b = O.uniform(n, 0x5EED0002, -1.0, 1.0)
    da, db, dc = up(a), up(b), empty(n)
    say("vecadd bench inputs n=2^24")
    kh.vecadd(da, db, dc, n)
    assert np.array_equal(down(dc, n), O.ref_vecadd(a, b))


def test_vecadd_wide_dynamic_range_correctly_rounded(dev):
    rng = np.random.default_rng(5)
    n = 1 << 18
    a = (rng.standard_normal(n) * 10.0 ** rng.integers(-30, 30, n)).astype(np.float32)
    b = (rng.standard_normal(n) * 10.0 ** rng.integers(-30, 30, n)).astype(np.float32)
    da, db, dc = up(a), up(b), empty(n)
    say("vecadd wide range")
    kh.vecadd(da, db, dc, n)
    assert np.array_equal(down(dc, n), O.ref_vecadd(a, b))


def test_vecadd_unaligned_and_offset_descriptors(dev):
    # Descriptors whose aligned pointer is 4 B past a 16 B boundary take the
    # scalar path; results must be identical.
    n = 10007
    a, b = O.vecadd_inputs(n + 1)
    da, db, dc = up(a), up(b), empty(n + 1)
    f = kh.template_function("vecadd")
    args = kh.LaunchArgs()
    for buf in (da, db, dc):
        args.add_memref(buf.ptr + 4, [n])
    say("vecadd unaligned")
    kh.kernel_launch(f, (7, 1, 1), (256, 1, 1), args)
    got = down(dc, n + 1)
    assert np.array_equal(got[1:], O.ref_vecadd(a[1:], b[1:]))


@pytest.mark.parametrize("n,dist", [(4194304, "lcg"), (1048576, "lcg"), (1000, "lcg"), (7, "lcg"),
                                    (1 << 22, "normal"), (1 << 26, "normal")])
def test_fused_gelu_vs_fp64_reference(dev, n, dist):
    seed = 0x3A5F91
    # The reference's own sizes use its LCG fill (U[-1,1) on a 2^-15 grid);
    # the BASELINE configurations 2^22 and 2^26 use N(0,1) inputs.
    x, _ = O.lcg_fill(n, seed) if dist == "lcg" else (O.normal(n, 0x6E1 + n, 0.0, 1.0), 0)
    dx, dtmp, do = up(x), empty(4, None), empty(n)
    say(f"fused_gelu n={n} {dist}")
    kh.fused_gelu(dx, dtmp, do, n)
    got = down(do, n).astype(np.float64)
    ref = O.ref_gelu(x)
    err = np.max(np.abs(got - ref))
    print(f"fused_gelu n={n} max-abs={err:.3e}")
    assert err <= 1e-4
    # Negative control (e2e_fused_gelu_test.cpp:307-382): no-tanh reference fails.
    assert np.max(np.abs(got - O.ref_gelu(x, with_tanh=False))) > 1e-4


def test_fused_gelu_extremes_finite(dev):
    # |x| up to 2e38 keeps t = 1.5x + 0.5 inside fp32 (beyond ~2.27e38 the
    # template's own fp32 fma overflows); t^3 overflowing must still give
    # gelu(t) = t for large positive t and 0 for large negative t.
    x = np.array([0.0, -1.0 / 3.0, 1e-30, -1e-30, 50.0, -50.0, 1e30, -1e30, 2e38, -2e38, 8.0, -8.0],
                 np.float32)
    n = x.size
    dx, do = up(x), empty(n)
    say("fused_gelu extremes")
    kh.fused_gelu(dx, dx, do, n)
    got = down(do, n).astype(np.float64)
    ref = O.ref_gelu(x)
    fin = np.isfinite(ref)
    assert np.all(np.abs(got[fin] - ref[fin]) <= 1e-4 + 1e-6 * np.abs(ref[fin]))
