"""kh_scan_noalloc (the allocation-free scan entry point) against kh_scan,
the entry point whose kernels it shares, on two calls in a row, the second
with a smaller input: bit-exact (inputs on a 2^-24 grid, so both equal the
fp64 prefix rounded to fp32). Plus the size limit, refused before any device
work."""
import numpy as np
import pytest

import kernelh as kh
import oracle as O
from khtest import down, empty, say, up


@pytest.mark.gpu
def test_scan_noalloc_matches_scan(dev):
    for call, n in enumerate((1 << 25, 1000003)):
        x = O.uniform(n, 0xA11C + n, 0.0, 1.0)
        T = kh.scan_workspace_floats(n)
        dx = up(x)
        ya, yb = empty(n), empty(n)
        say(f"scan_noalloc call={call} n={n}")
        kh.scan(dx, ya, empty(1, None), empty(T, None), empty(T, None), n)
        kh.scan_noalloc(dx, yb, n)
        a, b = down(ya, n), down(yb, n)
        assert np.array_equal(b, a), f"call {call}: {np.count_nonzero(a != b)} elements differ"
        assert np.array_equal(a, np.cumsum(x.astype(np.float64)).astype(np.float32))


def test_scan_noalloc_rejects_sizes_beyond_the_maximum():
    with pytest.raises(kh.KhrtError) as e:
        kh.scan_noalloc(0x1000, 0x2000, (1 << 31) + 1)
    assert e.value.code == kh.KHRT_E_INVALID and "exceeds the maximum of 2^31" in e.value.message
