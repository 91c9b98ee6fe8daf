"""fp32 MFMA GEMM on the GPU against the pinned oracle.

* Exact-integer fill (e2e_gemm_test.cpp:26-30, 70-75): products and K-deep
  sums are exact in fp32 for K <= 4096, so the result must be bit-exact at
  any accumulation order; sizes are the reference's {128, 512, 1024, 2048,
  4096, 1000}.
* BASELINE inputs U[-1,1]: relative Frobenius <= 1e-5 against the fp64
  reference (e2e_gemm_test.cpp:281); 8192^3 is checked on a row sample.
* Ragged shapes, the reference launch geometry, and the A*B^T negative
  control (e2e_gemm_test.cpp:289-375).
* Every tile symbol (`gemm` 128x256 persistent, `gemm_mid` 128x128,
  `gemm_wide` 128x128 persistent on 8 waves, `gemm_small` 64x64 persistent
  on 8 waves, `gemm_small_pf2` 64x64, `gemm_ksplit` and `gemm_ksplit_deep`
  32x32 with K split over the workgroup's waves, at any 64..512 threads)
  gives the same results at every shape and grid, whichever the launcher
  would pick; and the launcher's own grid (one workgroup per tile, or one
  round of resident workgroups for the persistent symbols; XCD-remapped)
  is checked at a shape it sends to each symbol.
"""
import json

import numpy as np
import pytest

import kernelh as kh
import oracle as O
from khtest import down, empty, say, up

pytestmark = pytest.mark.gpu


def _gemm(A, B, m, n, k):
    dA, dB, dC = up(A), up(B), empty(m * n)
    say(f"gemm m={m} n={n} k={k}")
    kh.gemm(dA, dB, dC, m, n, k)
    return down(dC, m * n).reshape(m, n)


@pytest.mark.parametrize("size", [128, 512, 1024, 2048, 4096, 1000])
def test_gemm_integer_fill_bit_exact(dev, size):
    A, B = O.gemm_int_inputs(size, size, size)
    C = _gemm(A, B, size, size, size)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)  # exact integers
    assert np.array_equal(C, ref)


@pytest.mark.parametrize("m,n,k", [(512, 512, 512), (2048, 2048, 2048), (8192, 8192, 256)])
def test_gemm_baseline_inputs_rel_frobenius(dev, m, n, k):
    A = O.uniform(m * k, 0xA11 + m, -1.0, 1.0).reshape(m, k)
    B = O.uniform(k * n, 0xB22 + n, -1.0, 1.0).reshape(k, n)
    C = _gemm(A, B, m, n, k)
    rows = np.arange(m) if m <= 2048 else np.arange(0, m, 97)
    ref = A[rows].astype(np.float64) @ B.astype(np.float64)
    err = O.rel_frobenius(C[rows], ref)
    print(f"gemm {m}x{n}x{k} rel-frobenius={err:.3e}")
    assert err <= 1e-5


def test_gemm_8192_cubed_row_sample(dev):
    m = n = k = 8192
    A = O.uniform(m * k, 0xA8192, -1.0, 1.0).reshape(m, k)
    B = O.uniform(k * n, 0xB8192, -1.0, 1.0).reshape(k, n)
    C = _gemm(A, B, m, n, k)
    # One row of every 128-row block (each row spans every column tile), at
    # an offset that varies from block to block, and the last row.
    blocks = np.arange(m // 128)
    rows = np.concatenate([blocks * 128 + (blocks * 53) % 128, [m - 1]])
    ref = A[rows].astype(np.float64) @ B.astype(np.float64)
    err = O.rel_frobenius(C[rows], ref)
    print(f"gemm 8192^3 rel-frobenius ({rows.size} rows, one per 128-row block)={err:.3e}")
    assert err <= 1e-5
    assert np.all(np.isfinite(C))


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (100, 37, 53), (129, 130, 131), (7, 1000, 3), (300, 5, 4097),
                                   (128, 256, 33), (255, 129, 64)])
def test_gemm_ragged_shapes(dev, m, n, k):
    A = O.uniform(m * k, 1, -1.0, 1.0).reshape(m, k)
    B = O.uniform(k * n, 2, -1.0, 1.0).reshape(k, n)
    C = _gemm(A, B, m, n, k)
    ref = O.ref_gemm(A, B, m, n, k)
    assert O.rel_frobenius(C, ref) <= 1e-5


def test_gemm_reference_geometry_and_negative_control(dev):
    m = n = k = 256
    A, B = O.gemm_int_inputs(m, n, k)
    dA, dB, dC = up(A), up(B), empty(m * n)
    f = kh.template_function("gemm")
    args = kh.LaunchArgs().add_memref(dA, [m, k]).add_memref(dB, [k, n]).add_memref(dC, [m, n])
    assert args.param_count() == 21
    say("gemm reference geometry ceil(m/32) x 256")
    kh.kernel_launch(f, ((m + 31) // 32, 1, 1), (256, 1, 1), args)
    C = down(dC, m * n).reshape(m, n)
    assert np.array_equal(C, O.ref_gemm(A, B, m, n, k).astype(np.float32))
    wrong = O.ref_gemm(A, B, m, n, k, transpose_b=True)
    assert O.rel_frobenius(C, wrong) > 1e-5


@pytest.mark.parametrize("symbol", ["gemm", "gemm_mid", "gemm_small", "gemm_small_pf2", "gemm_wide", "gemm_ksplit",
                                    "gemm_ksplit_deep"])
@pytest.mark.parametrize("m,n,k", [(256, 256, 256), (1000, 1000, 1000), (64, 192, 4097), (129, 65, 33),
                                   (3, 5, 7), (512, 2048, 96),
                                   # the sizes the launcher gives gemm_small_pf2 (>= 1024 tiles of 64x64),
                                   # with an odd slab count and a partial last slab, a short K, and an
                                   # unaligned K (generic path at 16-deep slabs).
                                   (2048, 2048, 260), (2112, 2048, 36), (2049, 2048, 33),
                                   # gemm's persistent cases: two slabs per tile (k = 20), one
                                   # slab (k = 16, its per-tile fallback), edge tiles in m and n.
                                   (300, 520, 20), (256, 512, 16), (1000, 1028, 100),
                                   # gemm's tail-free slab loads (K a multiple of 16, N of 256)
                                   # with edge tiles in m, and the smallest such K.
                                   (1000, 512, 64), (77, 256, 48), (520, 768, 32)])
def test_every_gemm_symbol_at_every_shape(dev, symbol, m, n, k):
    # Integer fill: exact in fp32, so both tilings must agree bit for bit.
    A, B = O.gemm_int_inputs(m, n, k) if k <= 4096 else (None, None)
    if A is None:
        A = O.uniform(m * k, 3, -1.0, 1.0).reshape(m, k)
        B = O.uniform(k * n, 4, -1.0, 1.0).reshape(k, n)
    mod = kh.GpuModule(kh.code_object("gemm"))
    f = mod.get_function(symbol)
    dA, dB, dC = up(A), up(B), empty(m * n)
    args = kh.LaunchArgs().add_memref(dA, [m, k]).add_memref(dB, [k, n]).add_memref(dC, [m, n])
    say(f"{symbol} m={m} n={n} k={k}")
    block = 512 if symbol in ("gemm_wide", "gemm_small") else 256  # their tile split is for 8 waves
    kh.kernel_launch(f, (37, 1, 1), (block, 1, 1), args)  # grid-strided: any grid
    C = down(dC, m * n).reshape(m, n)
    if k <= 4096:
        assert np.array_equal(C, (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))
    else:
        assert O.rel_frobenius(C, O.ref_gemm(A, B, m, n, k)) <= 1e-5


def test_gemm_symbols_random_shapes_exact(dev):
    """Seeded random shapes (ragged m, n, k; 60% with n, k multiples of 4 so
    the fast paths run) through every tile symbol at a random grid, with
    small-integer inputs: every sum is exact in fp32, so each result must
    equal the fp64 product bit for bit whatever the tiling and grid."""
    rng = np.random.default_rng(20261201)
    mod = kh.GpuModule(kh.code_object("gemm"))
    fns = {sym: mod.get_function(sym) for sym in ("gemm", "gemm_mid", "gemm_small", "gemm_small_pf2", "gemm_wide",
                                                       "gemm_ksplit", "gemm_ksplit_deep")}
    for _ in range(30):
        m, n = int(rng.integers(1, 700)), int(rng.integers(1, 700))
        k = int(rng.choice([int(rng.integers(1, 60)), int(rng.integers(1, 500))]))
        if rng.random() < 0.6:
            n, k = max(4, n // 4 * 4), max(4, k // 4 * 4)
        A = rng.integers(-3, 4, (m, k)).astype(np.float32)
        B = rng.integers(-3, 4, (k, n)).astype(np.float32)
        want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
        dA, dB, dC = up(A), up(B), empty(m * n)
        args = kh.LaunchArgs().add_memref(dA, [m, k]).add_memref(dB, [k, n]).add_memref(dC, [m, n])
        for sym, f in fns.items():
            grid = int(rng.choice([1, 3, 8, 37, 512]))
            block = (int(rng.choice([64, 192, 512])) if sym.startswith("gemm_ksplit")  # 1, 3 or 8 waves
                     else 512 if sym in ("gemm_wide", "gemm_small") else 256)
            say(f"{sym} m={m} n={n} k={k} grid={grid} block={block}")
            kh.kernel_launch(f, (grid, 1, 1), (block, 1, 1), args)
            assert np.array_equal(down(dC, m * n).reshape(m, n), want), (sym, m, n, k, grid)


@pytest.mark.parametrize("sym", ["gemm_ksplit", "gemm_ksplit_deep"])
@pytest.mark.parametrize("m,n,k,grid", [
    (32, 32, 128, 1),       # one tile, one batch per wave
    (96, 64, 384, 5),       # three batches per wave (an odd count)
    (512, 512, 512, 256),   # the BASELINE launch
    (256, 480, 1152, 37),   # 120 tiles over 37 workgroups
    (64, 2048, 2048, 64),   # deep K
    (512, 512, 192, 256),   # K not a multiple of 128: the general path
    (500, 512, 512, 256),   # M not a multiple of 32: the general path
])
def test_gemm_ksplit_interior_path(dev, sym, m, n, k, grid):
    """The K-split symbols at 512 threads on shapes whose tiles are all whole
    (M, N multiples of 32, K of 128: unconditional buffer loads), and on two
    that are not, with padded rows: A's rows k + 4 floats apart, B's n + 1,
    C's n + 3, every pad holding NaN. The result must equal the exact
    integer product bit for bit, and no pad may be read (NaN would reach C)
    or written."""
    lda, ldb, ldc = k + 4, n + 1, n + 3
    A, B = O.gemm_int_inputs(m, n, k)
    Ap = np.full((m, lda), np.nan, np.float32)
    Ap[:, :k] = A
    Bp = np.full((k, ldb), np.nan, np.float32)
    Bp[:, :n] = B
    dA, dB = up(Ap.ravel()), up(Bp.ravel())
    dC = up(np.full(m * ldc, np.nan, np.float32))
    args = kh.LaunchArgs().add_memref(dA, [m, k]).add_memref(dB, [k, n]).add_memref(dC, [m, n])
    args.slots[5], args.slots[7 + 5], args.slots[14 + 5] = lda, ldb, ldc
    f = kh.GpuModule(kh.code_object("gemm")).get_function(sym)
    say(f"{sym} m={m} n={n} k={k} grid={grid} block=512 lda={lda} ldb={ldb} ldc={ldc}")
    kh.kernel_launch(f, (grid, 1, 1), (512, 1, 1), args)
    C = down(dC, m * ldc).reshape(m, ldc)
    assert np.array_equal(C[:, :n], (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))
    assert np.isnan(C[:, n:]).all()


@pytest.mark.parametrize("extra", [4, 1])
def test_gemm_padded_c_rows(dev, extra):
    """C rows `n + extra` floats apart (slot 19 of the 21: C's row stride;
    16-byte aligned rows for extra = 4, not for extra = 1), through gemm's
    persistent path. The padding holds NaN and must stay NaN: no store
    lands past column n. m and n leave edge tiles in both dimensions; 5
    workgroups loop over 6 tiles."""
    m, n, k = 300, 520, 200
    pitch = n + extra
    A, B = O.gemm_int_inputs(m, n, k)
    dA, dB = up(A), up(B)
    dC = up(np.full(m * pitch, np.nan, np.float32))
    args = kh.LaunchArgs().add_memref(dA, [m, k]).add_memref(dB, [k, n]).add_memref(dC, [m, n])
    args.slots[14 + 5] = pitch
    mod = kh.GpuModule(kh.code_object("gemm"))
    f = mod.get_function("gemm")
    say(f"gemm m={m} n={n} k={k} C pitch={pitch}")
    kh.kernel_launch(f, (5, 1, 1), (256, 1, 1), args)
    C = down(dC, m * pitch).reshape(m, pitch)
    assert np.array_equal(C[:, :n], (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))
    assert np.isnan(C[:, n:]).all()


@pytest.mark.parametrize("m,n,k,grid", [
    (8192, 8192, 256, 512),     # gemm: 2048 tiles of 128x256 over 512 persistent workgroups
    (6144, 6144, 1024, 256),    # gemm_wide: 2304 tiles of 128x128 over 256 persistent workgroups
    (2048, 2048, 8192, 256),    # gemm_wide, deep K: one tile per workgroup
    (3072, 3072, 3072, 512),    # gemm_small: 2304 tiles of 64x64 over 512 persistent workgroups
    (8192, 1024, 8192, 256),    # gemm_wide: 512 tiles of 128x128, two per workgroup
    (4096, 4096, 4096, 512),    # gemm: one full round of 128x256
    (512, 512, 1024, 256),      # gemm_ksplit: 256 tiles of 32x32 at 512 threads
    (512, 470, 4100, 240),      # gemm_ksplit_deep: edge tiles in n, a partial last K chunk
    (768, 768, 768, 256),       # gemm_ksplit: 576 whole tiles of 32x32 looped over 256 workgroups
    (256, 2048, 2048, 256),     # gemm_ksplit_deep: 512 whole tiles looped
])
def test_gemm_launcher_choice_at_scale(dev, m, n, k, grid):
    assert kh.geometry("gemm", f"m={m},n={n},k={k}")[0] == (grid, 1, 1)
    rows = np.concatenate([np.arange(0, m, 61), [m - 1]])
    if k <= 4096:
        A, B = O.gemm_int_inputs(m, n, k)
        C = _gemm(A, B, m, n, k)
        ref = (A[rows].astype(np.float64) @ B.astype(np.float64)).astype(np.float32)  # exact integers
        assert np.array_equal(C[rows], ref)
    else:
        A = O.uniform(m * k, 0xC0 + m, -1.0, 1.0).reshape(m, k)
        B = O.uniform(k * n, 0xC1 + n, -1.0, 1.0).reshape(k, n)
        C = _gemm(A, B, m, n, k)
        err = O.rel_frobenius(C[rows], A[rows].astype(np.float64) @ B.astype(np.float64))
        print(f"gemm {m}x{n}x{k} rel-frobenius (rows sampled)={err:.3e}")
        assert err <= 1e-5


# ------------------------------------------------------------------ tune candidates

@pytest.mark.parametrize("m,n,k", [(200, 264, 72), (67, 45, 33), (129, 520, 260)])
def test_every_gemm_candidate_exact(dev, m, n, k):
    """Every GEMM candidate (the launcher's six symbols and the whole gfx950
    tune space: MFMA 32x32 and 16x16 tiles, 4 and 8 waves, every pipeline)
    at its own launch geometry, integer fill: bit-exact. (200, 264, 72) and
    (129, 520, 260) take the float4 paths with tails in m, n and k; (67, 45,
    33) the guarded generic path."""
    A, B = O.gemm_int_inputs(m, n, k)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    dA, dB, dC = up(A), up(B), empty(m * n)
    args = kh.LaunchArgs().add_memref(dA, [m, k]).add_memref(dB, [k, n]).add_memref(dC, [m, n])
    wrong = []
    for c in kh.gemm_candidates():
        sym = c["symbol"]
        grid, block = kh.gemm_candidate_geometry(sym, m, n, k)
        dC.fill(float("nan"))
        say(f"{sym} m={m} n={n} k={k} grid={grid} block={block}")
        kh.kernel_launch(kh.gemm_candidate_function(sym), grid, block, args)
        if not np.array_equal(down(dC, m * n).reshape(m, n), want):
            wrong.append(sym)
    assert not wrong, wrong


def test_tune_candidate_refuses_another_block_size(dev):
    # An 8-wave candidate launched with 256 threads writes NaN, never part
    # of the tile.
    m = n = k = 64
    A, B = O.gemm_int_inputs(m, n, k)
    dA, dB, dC = up(A), up(B), empty(m * n, 0.0)
    args = kh.LaunchArgs().add_memref(dA, [m, k]).add_memref(dB, [k, n]).add_memref(dC, [m, n])
    for sym in ("gemm_wide", next(c["symbol"] for c in kh.gemm_candidates() if c["waves"] == 8 and not c["product"])):
        dC.fill(0.0)
        say(f"{sym} at 256 threads (refused)")
        kh.kernel_launch(kh.gemm_candidate_function(sym), (4, 1, 1), (256, 1, 1), args)
        assert np.all(np.isnan(down(dC, m * n))), sym


@pytest.mark.parametrize("sym,block", [("gemm", 128), ("gemm_mid", 192), ("gemm_small", 256), ("gemm_small_pf2", 128)])
def test_product_symbols_refuse_another_block_size(dev, sym, block):
    # Each symbol's tile split assumes its own wave count (four; eight for
    # `gemm_small`): a smaller workgroup writes NaN over C, never part of
    # each tile. (A larger one is refused by the launch itself:
    # test_launch_above_the_kernel_bound_is_refused.)
    m = n = k = 64
    A, B = O.gemm_int_inputs(m, n, k)
    dA, dB, dC = up(A), up(B), empty(m * n, 0.0)
    args = kh.LaunchArgs().add_memref(dA, [m, k]).add_memref(dB, [k, n]).add_memref(dC, [m, n])
    say(f"{sym} at {block} threads (refused)")
    kh.kernel_launch(kh.gemm_candidate_function(sym), (4, 1, 1), (block, 1, 1), args)
    assert np.all(np.isnan(down(dC, m * n))), sym


def test_launch_above_the_kernel_bound_is_refused(dev):
    # A workgroup above the kernel's own bound (__launch_bounds__(256)) is
    # refused before it reaches the GPU, with the bound in the message.
    m = n = k = 64
    A, B = O.gemm_int_inputs(m, n, k)
    dA, dB, dC = up(A), up(B), empty(m * n, 0.0)
    args = kh.LaunchArgs().add_memref(dA, [m, k]).add_memref(dB, [k, n]).add_memref(dC, [m, n])
    f = kh.gemm_candidate_function("gemm")
    # The verifier alone first (nothing launched): only if it refuses is the
    # verified launch tried, which then refuses on the host the same way.
    diag = kh.verify_launch(512, grid=(4, 1, 1), function=f)
    assert "exceeds the kernel's own maximum 256" in diag, diag
    with pytest.raises(kh.KhrtError, match="exceeds the kernel's own maximum 256"):
        kh.kernel_launch(f, (4, 1, 1), (512, 1, 1), args)
    assert np.all(down(dC, m * n) == 0.0)


def test_tune_cache_steers_the_launcher(dev, tmp_path):
    """A tune cache entry for a shape makes kh_gemm (and the geometry and
    symbol queries) run the cached candidate for that shape only; other
    shapes keep the built-in choice; turning the cache off restores it."""
    m, n, k = 1000, 1000, 64
    shape = f"m={m},n={n},k={k}"
    pick = "gemm_m16_w2x4_t4x2_k16_p1_dma"  # 128 x 128 tiles, 8 waves, 16x16 MFMA
    default = kh.launch_symbol("gemm", shape)
    other = kh.launch_symbol("gemm", "m=1000,n=1000,k=68")
    assert default != pick
    cache = tmp_path / "tune-cache.json"
    cache.write_text(json.dumps({"key": kh.tune_cache_key("gemm", shape), "best": pick, "csv": ""}) + "\n")
    A, B = O.gemm_int_inputs(m, n, k)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    kh.set_tune_cache(str(cache))
    try:
        assert kh.launch_symbol("gemm", shape) == pick
        assert kh.geometry("gemm", shape) == kh.gemm_candidate_geometry(pick, m, n, k)
        assert kh.launch_symbol("gemm", "m=1000,n=1000,k=68") == other  # no entry: built-in choice
        C = _gemm(A, B, m, n, k)
        assert np.array_equal(C, want)
    finally:
        kh.set_tune_cache(None)
    assert kh.launch_symbol("gemm", shape) == default
