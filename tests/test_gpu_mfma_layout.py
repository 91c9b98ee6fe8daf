"""In-bounds check of the fp32 MFMA lane layouts the gemm and attention
kernels are written against (one wavefront, one instruction each):

v_mfma_f32_32x32x2f32   A: lane l holds A[i = l%32][k = l//32]
                        B: lane l holds B[k = l//32][j = l%32]
                        D: lane l, register r holds D[i][j] with
                           j = l%32, i = 8*(r//4) + 4*(l//32) + r%4
v_mfma_f32_16x16x4f32   A: A[l%16][l//16], B: B[l//16][l%16]
                        D: j = l%16, i = 4*(l//16) + r
"""
import os

import numpy as np
import pytest

import kernelh as kh
from khtest import down, say, up

pytestmark = pytest.mark.gpu


def _probe():
    with open(os.path.join(kh.CO_DIR, "mfma_probe.hsaco"), "rb") as f:
        return kh.GpuModule(f.read())


def _run(fn_name, a_lanes, b_lanes, regs):
    m = _probe()
    f = m.get_function(fn_name)
    da, db = up(a_lanes), up(b_lanes)
    out = kh.Buffer(64 * regs * 4)
    # Raw (unverified) launch: the probe takes plain pointers, not memrefs.
    args = kh.LaunchArgs()
    for buf in (da, db, out):
        args.slots.append(buf.ptr)
    say(f"mfma probe {fn_name}")
    kh.launch_raw(f, (1, 1, 1), (64, 1, 1), args)
    return down(out, 64 * regs).reshape(64, regs)


def test_mfma_32x32x2_f32_layout(dev):
    rng = np.random.default_rng(0)
    A = rng.integers(-8, 8, (32, 2)).astype(np.float32)
    B = rng.integers(-8, 8, (2, 32)).astype(np.float32)
    l = np.arange(64)
    a_lanes = A[l % 32, l // 32]
    b_lanes = B[l // 32, l % 32]
    D = A @ B
    got = _run("probe_mfma_32x32x2", a_lanes, b_lanes, 16)
    exp = np.empty((64, 16), np.float32)
    for lane in range(64):
        for r in range(16):
            exp[lane, r] = D[8 * (r // 4) + 4 * (lane // 32) + r % 4, lane % 32]
    assert np.array_equal(got, exp)


def test_mfma_16x16x4_f32_layout(dev):
    rng = np.random.default_rng(1)
    A = rng.integers(-8, 8, (16, 4)).astype(np.float32)
    B = rng.integers(-8, 8, (4, 16)).astype(np.float32)
    l = np.arange(64)
    D = A @ B
    got = _run("probe_mfma_16x16x4", A[l % 16, l // 16], B[l // 16, l % 16], 4)
    exp = np.empty((64, 4), np.float32)
    for lane in range(64):
        for r in range(4):
            exp[lane, r] = D[4 * (lane // 16) + r, lane % 16]
    assert np.array_equal(got, exp)
