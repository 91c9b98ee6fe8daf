"""The bench comparators (hipref-naive / hipref-vec, roofline_fma) compute
what they claim, so the CLI's comparator rows time correct kernels.

They mirror the reference's comparator set (bench/refs/*.hip, launched by
bench/harness/hipref_backend.cpp): raw-pointer ABIs, one workgroup per row
for softmax/layernorm, a two-pass scan, a 32x32 LDS-tiled GEMM. Checked
against the fp64 oracle with the reference's tolerances (1e-4 max abs for
softmax/layernorm/gelu; relative Frobenius 1e-5 for GEMM); the fp32 two-pass
scan to 1e-6 relative.
"""
import ctypes
import os

import numpy as np
import pytest

import kernelh as kh
import oracle as O
from khtest import down, empty, say, up

pytestmark = pytest.mark.gpu

HSACO = os.path.join(os.path.dirname(kh.LIB_PATH), "co", "hipref.hsaco")


@pytest.fixture(scope="module")
def mod(dev):
    return kh.GpuModule(open(HSACO, "rb").read())


def _args(*vals):
    a = kh.LaunchArgs()
    for v in vals:
        if isinstance(v, kh.Buffer):
            a.add_scalar_bytes(bytes(ctypes.c_uint64(v.ptr)))
        else:
            a.add_scalar_bytes(bytes(ctypes.c_int32(v)))
    return a


@pytest.mark.parametrize("variant", ["naive", "vec4"])
@pytest.mark.parametrize("rows,cols", [(64, 1024), (5, 4096), (3, 200)])
def test_softmax_and_layernorm_comparators(mod, variant, rows, cols):
    if variant == "vec4" and cols % 4:
        pytest.skip("vec4 needs cols % 4 == 0")
    x, seed = O.lcg_fill(rows * cols, 0x1234)
    g, seed = O.lcg_fill(cols, seed)
    b, seed = O.lcg_fill(cols, seed)
    dx, dy = up(x), empty(rows * cols)
    block = min(256, (min(cols, 256) + 63) // 64 * 64)
    say(f"softmax_{variant} {rows}x{cols}")
    kh.launch_raw(mod.get_function(f"softmax_{variant}"), (rows, 1, 1), (block, 1, 1), _args(dx, dy, rows, cols))
    assert np.max(np.abs(down(dy, rows * cols) - O.ref_softmax(x, rows, cols).ravel())) <= 1e-4
    dg, db = up(g), up(b)
    say(f"layernorm_{variant} {rows}x{cols}")
    kh.launch_raw(mod.get_function(f"layernorm_{variant}"), (rows, 1, 1), (256, 1, 1),
                  _args(dx, dg, db, dy, rows, cols))
    assert np.max(np.abs(down(dy, rows * cols) - O.ref_layernorm(x, g, b, rows, cols).ravel())) <= 1e-4


@pytest.mark.parametrize("variant", ["naive", "vec4"])
def test_fused_gelu_comparator(mod, variant):
    n = 100000
    x = O.normal(n, 0x6E1, 0.0, 1.0)
    dx, dy = up(x), empty(n)
    say(f"fused_gelu_{variant} n={n}")
    kh.launch_raw(mod.get_function(f"fused_gelu_{variant}"), ((n + 255) // 256, 1, 1), (256, 1, 1), _args(dx, dy, n))
    assert np.max(np.abs(down(dy, n) - O.ref_gelu(x))) <= 1e-4


@pytest.mark.parametrize("variant", ["naive", "vec4"])
@pytest.mark.parametrize("n", [100000, 1000, 4097])
def test_scan_comparator(mod, variant, n):
    x = O.uniform(n, 0x5CA + n, 0.0, 1.0)
    t = (n + 255) // 256
    dx, dy, dt = up(x), empty(n), empty(t)
    say(f"scan_{variant} n={n}")
    kh.launch_raw(mod.get_function(f"scan_pass1_{variant}"), (t, 1, 1), (256, 1, 1), _args(dx, dy, dt, n, t))
    kh.launch_raw(mod.get_function(f"scan_totals_{variant}"), (1, 1, 1), (256, 1, 1), _args(dt, dy, t, n))
    ref = O.ref_scan(x)
    got = down(dy, n)
    assert np.max(np.abs(got - ref) / np.maximum(ref, 1.0)) <= 1e-6


@pytest.mark.parametrize("m,n,k", [(128, 128, 128), (100, 70, 130), (33, 257, 5)])
def test_gemm_tiled_comparator(mod, m, n, k):
    A = O.uniform(m * k, 7, -1.0, 1.0)
    B = O.uniform(k * n, 8, -1.0, 1.0)
    dA, dB, dC = up(A), up(B), empty(m * n)
    say(f"gemm_tiled {m}x{n}x{k}")
    kh.launch_raw(mod.get_function("gemm_tiled"), ((n + 31) // 32, (m + 31) // 32, 1), (32, 8, 1),
                  _args(dA, dB, dC, m, n, k))
    assert O.rel_frobenius(down(dC, m * n).reshape(m, n), O.ref_gemm(A, B, m, n, k)) <= 1e-5


def test_roofline_fma_comparator(mod):
    n = 1 << 16
    dc = up(np.ones(n, np.float32))
    say("roofline_fma")
    kh.launch_raw(mod.get_function("roofline_fma"), (n // 256, 1, 1), (256, 1, 1), _args(dc, n, 64))
    got = down(dc, n)
    # 8 chains v_j = s + j, each 8 steps of v <- 0.999999 v + 1e-7.
    v = np.array([1.0 + j for j in range(8)], np.float64)
    for _ in range(8):
        v = v * 0.999999 + 1e-7
    assert np.allclose(got, v.sum(), rtol=1e-6)
