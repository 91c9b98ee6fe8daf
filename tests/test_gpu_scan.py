"""Single-pass look-back scan on the GPU: bit-exact against the fp64 prefix
rounded to fp32 (the reference pins max abs 0.0 at these sizes and seed,
e2e_scan_test.cpp:17-20, 225-256), the BASELINE sizes 10^6 and 2^26, ragged
tails, repeated calls on the same (dirty) buffers, and the exclusive-reference
negative control.

The reference launches `scan` and `scan_totals` itself, with plain
hipModuleLaunchKernel on uninitialised buffers and its own geometry
(kernelh_backend.cpp:334-357, e2e_scan_test.cpp:150-175). Those tests here go
through `khrt_launch_raw`: no verification, nothing launched before the
kernel, totals buffers as the caller left them (never written, zero-filled,
NaN-filled, or left by an earlier call or by the reference's own protocol).
"""
import os

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


def _scan_args(dx, dy, dylo, dth, dtl, n, T, T_hi=None, T_lo=None):
    a = kh.LaunchArgs().add_memref(dx, [n]).add_memref(dy, [n]).add_memref(dylo, [n]) \
        .add_memref(dth, [T if T_hi is None else T_hi]).add_memref(dtl, [T if T_lo is None else T_lo])
    assert a.param_count() == 25
    return a


def _raw_scan(f, x_buf, y_buf, ylo, th, tl, n, geometry):
    """One raw `scan` launch: the reference's geometry, ceil(n/256) x 256
    (kernelh_backend.cpp:335), or the launcher's (1024 threads, one resident
    round of workgroups)."""
    T = kh.scan_workspace_floats(n)
    if geometry == "reference":
        grid, block = (T, 1, 1), (256, 1, 1)
    else:
        grid, block = kh.geometry("scan", f"n={n}")
        grid = (min(grid[0], 256), 1, 1)
    kh.launch_raw(f, grid, block, _scan_args(x_buf, y_buf, ylo, th, tl, n, T))


# What the caller's totals buffers hold before the first launch.
_TOTALS = {"uninitialised": None, "zero": 0.0, "nan": float("nan"), "ones": 1.0}


@pytest.mark.parametrize("n", [1000000, 1 << 26])
@pytest.mark.parametrize("geometry", ["reference", "launcher"])
def test_scan_raw_launch_any_totals(dev, n, geometry):
    """`scan` alone through plain hipModuleLaunchKernel on totals in every
    starting state, then again on the same buffers (state left by the
    previous call), bit-exact each time."""
    x = O.uniform(n, 0x5CA4 + n, 0.0, 1.0)  # 2^-24 grid: the fp64 prefix is exact
    ref = np.cumsum(x.astype(np.float64)).astype(np.float32)
    T = kh.scan_workspace_floats(n)
    m = kh.GpuModule(kh.code_object("scan"))
    f = m.get_function("scan")
    dx = up(x)
    for state, fill in _TOTALS.items():
        th, tl = empty(T, fill), empty(T, fill)
        for call in range(2):
            dy = empty(n)
            say(f"scan raw n={n} geometry={geometry} totals={state} call={call}")
            _raw_scan(f, dx, dy, empty(1, None), th, tl, n, geometry)
            got = down(dy, n)
            bad = np.flatnonzero(got != ref)
            assert bad.size == 0, f"{state} call {call}: {bad.size} differ, first at {bad[:5]}"


def test_scan_raw_launch_misaligned_totals(dev):
    """Totals descriptors that start 4 bytes past an 8-byte boundary (the
    header and records move to the next boundary inside the buffer)."""
    n = 500000
    T = kh.scan_workspace_floats(n)
    x = O.mt19937_fill(n, 0x29C0FFEE)
    ref = O.ref_scan(x)
    f = kh.GpuModule(kh.code_object("scan")).get_function("scan")
    th_big, tl_big = empty(T + 2, 3.0), empty(T + 2, -2.0)
    dx = up(x)
    for call in range(2):
        dy = empty(n)
        say(f"scan raw misaligned totals call={call}")
        kh.launch_raw(f, (T, 1, 1), (256, 1, 1),
                      _scan_args(dx, dy, empty(1, None), th_big.ptr + 4, tl_big.ptr + 4, n, T))
        assert np.array_equal(down(dy, n), ref)


def test_scan_reference_two_launch_protocol(dev):
    # Raw protocol: caller geometry ceil(n/256) x 256 for `scan`, 1 x 256 for
    # `scan_totals`, uninitialised device buffers, plain launches; then a
    # second scan on the same buffers after scan_totals has run.
    n = 65536 + 17
    T = (n + 255) // 256
    x = O.mt19937_fill(n, 0x29C0FFEE)
    dx = up(x)
    dy, dylo = empty(n), empty(n, None)
    dth, dtl, oh, ol, ol2 = (empty(T, None) for _ in range(5))
    m = kh.GpuModule(kh.code_object("scan"))
    f1, f2 = m.get_function("scan"), m.get_function("scan_totals")
    a2 = kh.LaunchArgs()
    for b, s in ((dth, T), (dtl, T), (oh, T), (ol, T), (ol2, T), (dy, n), (dylo, n)):
        a2.add_memref(b, [s])
    assert a2.param_count() == 35
    ref = O.ref_scan(x)
    for call in range(2):
        dy.fill(float("nan"))
        say(f"scan raw two-launch protocol call={call}")
        kh.launch_raw(f1, (T, 1, 1), (256, 1, 1), _scan_args(dx, dy, dylo, dth, dtl, n, T))
        kh.launch_raw(f2, (1, 1, 1), (256, 1, 1), a2)
        got = down(dy, n)
        assert np.array_equal(got, ref)
        offs = down(oh, T)
        assert offs[0] == 0.0 and np.array_equal(offs[1:], ref[255:-1:256][: T - 1])


def test_scan_verified_kernel_launch(dev):
    # The reference's KernelLaunch path (verified, then launched) on the
    # same code object, reference geometry.
    n = 123457
    T = kh.scan_workspace_floats(n)
    x = O.mt19937_fill(n, 0x51AC0D3E)
    f = kh.GpuModule(kh.code_object("scan")).get_function("scan")
    dy = empty(n)
    say("scan verified kernel_launch")
    kh.kernel_launch(f, (T, 1, 1), (256, 1, 1), _scan_args(up(x), dy, empty(1, None), empty(T, None),
                                                           empty(T, None), n, T))
    assert np.array_equal(down(dy, n), O.ref_scan(x))


@pytest.mark.parametrize("short", ["totals_hi", "totals_lo", "block"])
def test_scan_refuses_without_touching_totals(dev, short):
    """Too little room for the look-back state, or a workgroup shape the tile
    loop does not take: y becomes NaN and the totals (and the memory past
    them) keep their contents."""
    n = 200000  # 66 tiles of 3072 at 256 threads: 65 records of 16 B = 260 floats
    T = kh.scan_workspace_floats(n)
    x = O.uniform(n, 5, 0.0, 1.0)
    guard = 4096
    th, tl = empty(T + guard, 5.0), empty(T + guard, 6.0)
    t_hi, t_lo, block = T, T, 256
    if short == "totals_hi":
        t_hi = 200
    elif short == "totals_lo":
        t_lo = 9  # 36 B: the 32-byte header and 16 B of counters (48 B) do not fit
    else:
        block = 128
    f = kh.GpuModule(kh.code_object("scan")).get_function("scan")
    dy = empty(n, 0.25)
    say(f"scan refusal short={short}")
    kh.launch_raw(f, ((n + block - 1) // block, 1, 1), (block, 1, 1),
                  _scan_args(up(x), dy, empty(1, None), th, tl, n, T, t_hi, t_lo))
    assert np.all(np.isnan(down(dy, n)))
    assert np.all(down(th, T + guard) == 5.0) and np.all(down(tl, T + guard) == 6.0)


def test_scan_two_streams_distinct_buffers(dev):
    """Calls on different totals buffers are independent, also when they run
    at the same time on two streams."""
    n = 1 << 22
    xs = [O.uniform(n, 900 + i, 0.0, 1.0) for i in range(2)]
    refs = [np.cumsum(x.astype(np.float64)).astype(np.float32) for x in xs]
    T = kh.scan_workspace_floats(n)
    streams = [kh.Stream(), kh.Stream()]
    bufs = [(up(x), empty(n), empty(1, None), empty(T, None), empty(T, None)) for x in xs]
    for rep in range(3):
        say(f"scan two streams rep={rep}")
        for (dx, dy, dylo, th, tl), s in zip(bufs, streams):
            kh.scan(dx, dy, dylo, th, tl, n, s)
        for s in streams:
            s.synchronize()
        for (dx, dy, *_), ref in zip(bufs, refs):
            assert np.array_equal(down(dy, n), ref)
    for s in streams:
        s.destroy()


def test_scan_negative_control_exclusive(dev):
    n = 1024
    x = O.mt19937_fill(n, 0x51AC0D3E)
    got, _ = _scan(x, n)
    assert np.max(np.abs(got.astype(np.float64) - O.ref_scan(x, exclusive=True))) > 1e-4


# Off the grid: inputs whose partial sums fp64 cannot hold exactly. y is then
# fl32 of an fp64 tree sum, not always the correctly rounded prefix r. Every
# fp64 partial sum S_i is a sum of the x_j (j <= i) through a tree in which no
# input passes more than D additions, so |S_i - P_i| <= gamma_D A_i, with P_i
# the exact prefix, A_i = sum |x_j| and gamma_D = D u/(1 - D u), u = 2^-53
# (Higham, Accuracy and Stability of Numerical Algorithms, 2nd ed., 4.2).
# Rounding both S_i and P_i to fp32 (unit 2^-24) gives
#     |y_i - r_i| <= 2^-23 |r_i| / (1 - 2^-24) + (1 + 2^-24) gamma_D A_i.
# D for this kernel: an element passes 3 additions into its float4 row sum,
# 6 in the wave's DPP scan, 1 in `inc - sk`, 4 over its wave's rows, 14 over
# earlier waves, 6 in the tile aggregate, 4 in its own float4, 2 with the
# prefix; a tile's inclusive prefix adds at most 1 + 6 + (windows walked) to
# its nearest published predecessor's, which in the worst case is the tile
# just before it. D = 10 ntiles + 64 bounds all of this; ntiles is counted
# for the smallest tile the kernel accepts (256-thread workgroups: 3 data
# waves x 64 lanes x 16 elements), so the bound holds for any launch shape.
def _offgrid(kind, n):
    rng = np.random.default_rng(0x0FF6)
    x = rng.standard_normal(n)
    if kind == "wide":
        x = x * np.exp2(rng.integers(-20, 21, n).astype(np.float64))
    return x.astype(np.float32)


@pytest.mark.parametrize("kind", ["normal", "wide"])
def test_scan_off_grid_inputs_within_derived_bound(dev, kind):
    n = 1 << 20
    x = _offgrid(kind, n)
    got, _ = _scan(x, n)
    r, A, margin = O.ref_scan_exact(x, with_abs=True, with_margin=True)
    tile = 3 * 64 * 16
    D = 10 * ((n + tile - 1) // tile) + 64
    u = 2.0 ** -53
    gamma = D * u / (1 - D * u)
    r64 = r.astype(np.float64)
    tol = 2.0 ** -23 * np.abs(r64) / (1 - 2.0 ** -24) + (1 + 2.0 ** -24) * gamma * A
    err = np.abs(got.astype(np.float64) - r64)
    assert np.all(np.isfinite(got))
    worst = int(np.argmax(err / tol))
    # Where the exact prefix lies farther from every fp32 rounding boundary
    # than the fp64 sum can stray (gamma_D A_i, plus the margin's own fp64
    # error), the fp64 sum rounds to the same fp32 value: y must equal the
    # correctly rounded prefix exactly there. Only the rest may differ.
    forced = margin > gamma * A + 2.0 ** -50 * np.abs(r64)
    differ = got != r
    emu = O.emu_scan_template(x)
    say(f"scan off-grid {kind}: {int(np.sum(differ))} of {n} differ from the correctly rounded prefix "
        f"({int(np.sum(~forced))} lie within the bound of a rounding boundary), {int(np.sum(emu != r))} for the "
        f"template emulator; worst err/tol {err[worst] / tol[worst]:.3g} at {worst}")
    assert np.all(err <= tol), f"element {worst}: |y - r| = {err[worst]:.3e} > {tol[worst]:.3e}"
    bad = np.flatnonzero(differ & forced)
    assert bad.size == 0, f"{bad.size} elements differ where the bound forces the correct rounding: {bad[:5]}"
    # The check is not vacuous: the bound leaves 2.8% (normal) and 0.8%
    # (wide) of these inputs' prefixes near enough a boundary to go either way.
    assert int(np.sum(forced)) >= n - n // 20


# The look-back state's layout and hashes, restated on the host so that a
# test can forge states the kernel must survive (scan.hip: Header, Counters,
# mix64, header_check, claim_mark). totals_lo holds, from its first 8-byte
# boundary, base (u64: generation << 32 | first ticket), nonce (u64), check
# (u64), failed (u32), pad; the ticket counter (u32), pad and done (u64) sit
# 256 B further on when totals_lo has room.
_M64 = (1 << 64) - 1


def _mix64(z):
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def _header_check(h, base, nonce):
    key = _mix64(h ^ _mix64(nonce ^ 0x5CA11AB1E5CA4A11))
    return _mix64(key ^ _mix64(base ^ 0x0C0FFEE0DDBA11)) or 1


def _claim_mark(h):
    return _mix64(h ^ 0xC1A1BEDC1A1BED) & ~0xFF & _M64


def _forge_totals_lo(buf, T, base, nonce, check, counter, failed=0, done=0):
    assert buf.ptr % 8 == 0 and 4 * T >= 256 + 16
    w = np.zeros(T, np.uint32)
    w64 = w[:8].view(np.uint64)
    w64[0], w64[1], w64[2] = base, nonce, check
    w[6] = failed
    w[64] = counter
    w[66:68].view(np.uint64)[0] = done
    buf.copy_from_host(w)


def _failed(buf):
    return int(buf.to_host(np.uint32, 8)[6])


def _shortspin_scan():
    with open(os.path.join(kh.CO_DIR, "scan_shortspin.hsaco"), "rb") as f:
        m = kh.GpuModule(f.read())
    return m, m.get_function("scan")


def test_scan_lookback_gives_up_on_a_missing_record(dev):
    """A signed header whose counter skips tile 0's ticket: tile 0 is never
    handed out, so tile 1's look-back waits for a record that never comes.
    (Half as many workgroups as tiles, so that tiles go by ticket.)
    With the test build's short bounded wait it gives up: every later tile
    is NaN, tile 0's elements are untouched, the header counts the failure,
    every workgroup exits, and the call still closes, so the next call on
    the same buffers (the product code object) is bit-exact."""
    n = 10 ** 6
    T = kh.scan_workspace_floats(n)
    tile = 15 * 64 * 16  # 1024-thread workgroups: 15 data waves x 64 lanes x 16
    ntiles = (n + tile - 1) // tile
    x = O.uniform(n, 0x6173, 0.0, 1.0)
    ref = np.cumsum(x.astype(np.float64)).astype(np.float32)
    dx, th, tl = up(x), empty(T, 0.0), empty(T, 0.0)
    first = 5000
    base, nonce = (7 << 32) | first, 0x123456789ABC
    _forge_totals_lo(tl, T, base, nonce, _header_check(tl.ptr, base, nonce), counter=first + 1)
    _m, f = _shortspin_scan()
    dy = empty(n, 0.25)
    grid = ntiles // 2
    say(f"scan short-spin look-back give-up n={n} grid={grid}x1024")
    kh.launch_raw(f, (grid, 1, 1), (1024, 1, 1), _scan_args(dx, dy, empty(1, None), th, tl, n, T))
    got = down(dy, n)
    assert np.all(got[:tile] == 0.25)
    assert np.all(np.isnan(got[tile:]))
    assert _failed(tl) >= 1
    g = kh.GpuModule(kh.code_object("scan")).get_function("scan")
    for grid in (ntiles // 2, ntiles):  # tiles by ticket, then by workgroup index
        dy = empty(n)
        say(f"scan after a give-up: same buffers, product code object, grid={grid}")
        kh.launch_raw(g, (grid, 1, 1), (1024, 1, 1), _scan_args(dx, dy, empty(1, None), th, tl, n, T))
        assert np.array_equal(down(dy, n), ref)


def test_scan_takes_over_a_stale_claim(dev):
    """A header that holds a claim mark when the call begins (a claim that
    never signs): after the bounded wait one workgroup takes the claim over
    under the next epoch's mark, so the call is bit-exact with no failure
    counted, and so is the next one."""
    n = 10 ** 6
    T = kh.scan_workspace_floats(n)
    x = O.uniform(n, 0x6174, 0.0, 1.0)
    ref = np.cumsum(x.astype(np.float64)).astype(np.float32)
    dx, th, tl = up(x), empty(T, 3.0), empty(T, 0.0)
    _forge_totals_lo(tl, T, base=12345, nonce=99, check=_claim_mark(tl.ptr) | 5, counter=777, failed=0, done=31)
    _m, f = _shortspin_scan()
    for call in range(2):
        dy = empty(n)
        say(f"scan short-spin stale claim call={call}")
        kh.launch_raw(f, (66, 1, 1), (1024, 1, 1), _scan_args(dx, dy, empty(1, None), th, tl, n, T))
        assert np.array_equal(down(dy, n), ref)
        assert _failed(tl) == 0
