"""Fused fp32 MFMA attention on the GPU against the fp64 reference rows.

Tolerance: every element |g - r| <= 2e-3 + 2e-3 |r| (e2e_attention_test.cpp:
298-311). Covers the reference's e2e shape (b=2, h=8, s in {512, 1024},
LCG seeds 0x313A171B / 0x51AC0D3E / 0x29C0FFEE, attention_test.cpp:64-79,
all rows), the BASELINE shapes b=4, h=16, s in {1024, 4096} with N(0,1)
inputs (row sample), ragged sequence lengths, the reference launch geometry
and the no-1/sqrt(d) negative control (e2e_attention_test.cpp:319-348).
"""
import numpy as np
import pytest

import kernelh as kh
import oracle as O
from khtest import down, empty, say, up

pytestmark = pytest.mark.gpu
D = 64


def _attention(Q, K, V, b, h, s):
    n = b * h * s * D
    dq, dk, dv, do = up(Q), up(K), up(V), empty(n)
    say(f"attention b={b} h={h} s={s}")
    kh.attention(dq, dk, dv, do, b, h, s, D)
    return down(do, n).reshape(b * h, s, D)


def _rows(b, h, s, count, seed):
    if count is None:
        return np.repeat(np.arange(b * h), s), np.tile(np.arange(s), b * h)
    rng = np.random.default_rng(seed)
    bh = rng.integers(0, b * h, count)
    qi = rng.integers(0, s, count)
    bh[:2], qi[:2] = [0, b * h - 1], [0, s - 1]
    return bh, qi


def _check(Q, K, V, got, b, h, s, count=None, seed=0):
    bh, qi = _rows(b, h, s, count, seed)
    ref = O.ref_attention_rows(Q, K, V, s, D, bh, qi)
    g = got[bh, qi]
    viol = O.attention_violation(g, ref)
    print(f"attention b={b} h={h} s={s} rows={bh.size} max-abs={np.max(np.abs(g - ref)):.3e} viol={viol:.3e}")
    assert np.all(np.isfinite(g))
    assert viol <= 2e-3
    return g, ref, bh, qi


@pytest.mark.parametrize("s", [512, 1024])
def test_attention_reference_e2e_shape_all_rows(dev, s):
    b, h = 2, 8
    n = b * h * s * D
    Q, _ = O.lcg_fill(n, 0x313A171B)
    K, _ = O.lcg_fill(n, 0x51AC0D3E)
    V, _ = O.lcg_fill(n, 0x29C0FFEE)
    O.set_threads(8)
    _check(Q, K, V, _attention(Q, K, V, b, h, s), b, h, s)


@pytest.mark.parametrize("s", [1024, 4096])
def test_attention_baseline_shapes(dev, s):
    """The BASELINE shapes: every query row at s = 1024; at s = 4096 (a
    quarter of a million rows, too many for the fp64 reference in seconds)
    one row of every 128-row query tile of every slice, at an offset that
    varies from tile to tile, so every workgroup's output is checked."""
    b, h = 4, 16
    n = b * h * s * D
    Q = O.normal(n, 0xA1, 0.0, 1.0)
    K = O.normal(n, 0xA2, 0.0, 1.0)
    V = O.normal(n, 0xA3, 0.0, 1.0)
    O.set_threads(16)
    got = _attention(Q, K, V, b, h, s)
    if s <= 1024:
        _check(Q, K, V, got, b, h, s)
        return
    tiles = s // 128
    bh = np.repeat(np.arange(b * h), tiles)
    t = np.tile(np.arange(tiles), b * h)
    qi = t * 128 + (t * 53 + bh * 29) % 128
    ref = O.ref_attention_rows(Q, K, V, s, D, bh, qi)
    g = got[bh, qi]
    viol = O.attention_violation(g, ref)
    print(f"attention b={b} h={h} s={s} rows={bh.size} (one per query tile) viol={viol:.3e}")
    assert np.all(np.isfinite(g)) and viol <= 2e-3


@pytest.mark.parametrize("b,h,s", [(1, 1, 1), (1, 2, 100), (2, 3, 67), (1, 1, 129), (3, 1, 200)])
def test_attention_ragged_sequences(dev, b, h, s):
    n = b * h * s * D
    Q = O.normal(n, 1, 0.0, 1.0)
    K = O.normal(n, 2, 0.0, 1.0)
    V = O.normal(n, 3, 0.0, 1.0)
    _check(Q, K, V, _attention(Q, K, V, b, h, s), b, h, s)


@pytest.mark.parametrize("pitch", [80, 68, 66])
def test_attention_padded_row_stride(dev, pitch):
    """[b, h, s, d] slices whose rows are `pitch` floats apart (d = 64 used):
    the kernel takes the row stride from the memref (attention.cpp reads
    s2 through the descriptor). 80 and 68 keep rows 16-byte aligned (the
    pipelined float4 path); 66 does not (the element-wise path). The padding
    holds NaN, so a read past a row's 64 floats shows up as a non-finite
    output."""
    b, h, s = 2, 2, 200
    n = b * h * s * D
    Q = O.normal(n, 11, 0.0, 1.0)
    K = O.normal(n, 12, 0.0, 1.0)
    V = O.normal(n, 13, 0.0, 1.0)

    def padded(x):
        p = np.full((b * h * s, pitch), np.nan, np.float32)
        p[:, :D] = x.reshape(b * h * s, D)
        return up(p.ravel())

    dq, dk, dv, do = padded(Q), padded(K), padded(V), up(np.zeros(b * h * s * pitch, np.float32))
    args = kh.LaunchArgs()
    for buf in (dq, dk, dv, do):
        args.add_memref(buf, [b, h, s, D])
    # Rank-4 descriptor: ptr, ptr, offset, 4 sizes, 4 strides (slots 7..10).
    for i in range(4):
        base = 11 * i
        args.slots[base + 7:base + 11] = [h * s * pitch, s * pitch, pitch, 1]
    say(f"attention padded rows pitch={pitch} b={b} h={h} s={s}")
    kh.kernel_launch(kh.template_function("attention"), ((s + 127) // 128, h, b), (256, 1, 1), args)
    got = down(do, b * h * s * pitch).reshape(b * h, s, pitch)[:, :, :D]
    _check(Q, K, V, np.ascontiguousarray(got), b, h, s)


@pytest.mark.parametrize("threads", [256, 64])
def test_attention_distinct_pitches(dev, threads):
    """Q, K, V and O each with a row pitch of their own (64 / 68 / 80 / 72
    floats; 256-thread workgroups take the pipelined path, 64-thread ones
    the synchronous one). Padding is NaN in the inputs, so reading V (or K)
    with another tensor's stride shows up as a wrong or non-finite row; O's
    padding must keep its sentinel."""
    b, h, s = 2, 2, 200
    pitches = {"Q": 64, "K": 68, "V": 80, "O": 72}
    n = b * h * s * D
    Q = O.normal(n, 21, 0.0, 1.0)
    K = O.normal(n, 22, 0.0, 1.0)
    V = O.normal(n, 23, 0.0, 1.0)

    def padded(x, pitch, fill):
        p = np.full((b * h * s, pitch), fill, np.float32)
        if x is not None:
            p[:, :D] = x.reshape(b * h * s, D)
        return p

    host = {"Q": padded(Q, 64, np.nan), "K": padded(K, 68, np.nan), "V": padded(V, 80, np.nan),
            "O": padded(None, 72, -7.0)}
    bufs = {k: up(v.ravel()) for k, v in host.items()}
    args = kh.LaunchArgs()
    for i, name in enumerate(("Q", "K", "V", "O")):
        p = pitches[name]
        args.add_memref(bufs[name], [b, h, s, D])
        # Rank-4 descriptor: ptr, ptr, offset, 4 sizes, 4 strides (slots 7..10).
        args.slots[11 * i + 7:11 * i + 11] = [h * s * p, s * p, p, 1]
    say(f"attention distinct pitches {pitches} threads={threads}")
    grid = ((s + 127) // 128, h, b) if threads == 256 else (s, h, b)
    kh.kernel_launch(kh.template_function("attention"), grid, (threads, 1, 1), args)
    out = down(bufs["O"], b * h * s * 72).reshape(b * h * s, 72)
    assert np.all(out[:, D:] == -7.0), "O's row padding was written"
    _check(Q, K, V, np.ascontiguousarray(out[:, :D]).reshape(b * h, s, D), b, h, s)


@pytest.mark.parametrize("bad", ["head_dim32", "kv_seq", "v_heads"])
def test_attention_refuses_other_shapes(dev, bad):
    """head_dim != 64 (attention.cpp:115-120) or K/V extents that differ from
    Q's: O is filled with NaN (by its own descriptor) and nothing past it is
    touched."""
    b, h, s, d = 1, 2, 128, 64
    shapes = {k: [b, h, s, d] for k in "QKVO"}
    if bad == "head_dim32":
        shapes = {k: [b, h, s, 32] for k in "QKVO"}
    elif bad == "kv_seq":
        shapes["K"] = [b, h, s // 2, d]
        shapes["V"] = [b, h, s // 2, d]
    else:
        shapes["V"] = [b, 1, s, d]
    guard = 1024
    bufs = {k: empty(int(np.prod(v)) + guard, 1.0) for k, v in shapes.items()}
    args = kh.LaunchArgs()
    for k in "QKVO":
        args.add_memref(bufs[k], shapes[k])
    say(f"attention refusal {bad}")
    kh.launch_raw(kh.template_function("attention"), ((s + 127) // 128, h, b), (256, 1, 1), args)
    no = int(np.prod(shapes["O"]))
    out = down(bufs["O"], no + guard)
    assert np.all(np.isnan(out[:no])) and np.all(out[no:] == 1.0)


def test_attention_reference_geometry_and_negative_control(dev):
    b, h, s = 1, 2, 256
    n = b * h * s * D
    Q, _ = O.lcg_fill(n, 0x313A171B)
    K, _ = O.lcg_fill(n, 0x51AC0D3E)
    V, _ = O.lcg_fill(n, 0x29C0FFEE)
    dq, dk, dv, do = up(Q), up(K), up(V), empty(n)
    f = kh.template_function("attention")
    args = kh.LaunchArgs()
    for buf in (dq, dk, dv, do):
        args.add_memref(buf, [b, h, s, D])
    assert args.param_count() == 44
    say("attention reference geometry (seq, heads, batch) x 64")
    kh.kernel_launch(f, (s, h, b), (64, 1, 1), args)
    got = down(do, n).reshape(b * h, s, D)
    g, ref, bh, qi = _check(Q, K, V, got, b, h, s)
    wrong = O.ref_attention_rows(Q, K, V, s, D, bh, qi, scaled=False)
    assert O.attention_violation(g, wrong) > 2e-3
