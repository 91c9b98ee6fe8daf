"""Single-pass look-back scan on the GPU: bit-exact against the fp64 prefix
rounded to fp32 (the reference pins max abs 0.0 at these sizes and seed,
e2e_scan_test.cpp:17-20, 225-256), the BASELINE sizes 10^6 and 2^26, ragged
tails, repeated calls on the same (dirty) buffers, the reference's raw
two-launch protocol (scan then scan_totals on uninitialised buffers,
kernelh_backend.cpp:334-357) and the exclusive-reference negative control.
"""
import numpy as np
import pytest

import kernelh as kh
import oracle as O
from khtest import down, empty, say, up

pytestmark = pytest.mark.gpu


def _scan(x, n, bufs=None):
    T = kh.scan_workspace_floats(n)
    if bufs is None:
        bufs = (up(x), empty(n), empty(n, None), empty(T, 1234.5), empty(T, 7.0))
    dx, dy, dylo, dth, dtl = bufs
    say(f"scan n={n}")
    kh.scan(dx, dy, dylo, dth, dtl, n)
    return down(dy, n), bufs


@pytest.mark.parametrize("n", [1024, 65536, 1 << 20, 1000, 1, 4095, 4096, 4097, 8193, 1000000])
def test_scan_bit_exact_reference_seed(dev, n):
    x = O.mt19937_fill(n, 0x29C0FFEE)
    got, _ = _scan(x, n)
    ref = O.ref_scan(x)
    assert np.array_equal(got, ref), f"max abs {np.max(np.abs(got.astype(np.float64) - ref))}"


def test_scan_bit_exact_baseline_2_26(dev):
    n = 1 << 26
    x = O.uniform(n, 0x5CA4, 0.0, 1.0)  # 2^-24 grid: the fp64 prefix is exact
    got, _ = _scan(x, n)
    ref = np.cumsum(x.astype(np.float64)).astype(np.float32)
    assert np.array_equal(got, ref)


def test_scan_repeated_calls_reuse_state(dev):
    n = 300000
    x = O.uniform(n, 77, 0.0, 1.0)
    got, bufs = _scan(x, n)
    ref = O.ref_scan(x)
    assert np.array_equal(got, ref)
    for _ in range(3):
        got, _ = _scan(x, n, bufs)
        assert np.array_equal(got, ref)


def test_scan_reference_two_launch_protocol(dev):
    # Raw protocol: caller geometry ceil(n/256) x 256 for `scan`, 1 x 256 for
    # `scan_totals`, uninitialised device buffers, verified KernelLaunch path.
    n = 65536 + 17
    T = (n + 255) // 256
    x = O.mt19937_fill(n, 0x29C0FFEE)
    dx = up(x)
    dy, dylo = empty(n), empty(n, None)
    dth, dtl, oh, ol, ol2 = (empty(T, None) for _ in range(5))
    m = kh.GpuModule(kh.code_object("scan"))
    f1, f2 = m.get_function("scan"), m.get_function("scan_totals")
    a1 = kh.LaunchArgs().add_memref(dx, [n]).add_memref(dy, [n]).add_memref(dylo, [n]) \
        .add_memref(dth, [T]).add_memref(dtl, [T])
    assert a1.param_count() == 25
    a2 = kh.LaunchArgs()
    for b, s in ((dth, T), (dtl, T), (oh, T), (ol, T), (ol2, T), (dy, n), (dylo, n)):
        a2.add_memref(b, [s])
    assert a2.param_count() == 35
    say("scan raw two-launch protocol")
    kh.kernel_launch(f1, (T, 1, 1), (256, 1, 1), a1)
    kh.kernel_launch(f2, (1, 1, 1), (256, 1, 1), a2)
    got = down(dy, n)
    ref = O.ref_scan(x)
    assert np.array_equal(got, ref)
    offs = down(oh, T)
    assert offs[0] == 0.0 and np.array_equal(offs[1:], ref[255:-1:256][: T - 1])


def test_scan_negative_control_exclusive(dev):
    n = 1024
    x = O.mt19937_fill(n, 0x51AC0D3E)
    got, _ = _scan(x, n)
    assert np.max(np.abs(got.astype(np.float64) - O.ref_scan(x, exclusive=True))) > 1e-4
