"""softmax and layernorm on the GPU against the pinned fp64 references.

Tolerance: max abs <= 1e-4 (e2e_softmax_test.cpp:308, e2e_layernorm_test.cpp:
320). Shapes: the reference's {(4096,1024), (16384,4096), (1,8192)}, the
BASELINE inputs (N(0, 4^2) rows; gamma U[0.5,1.5], beta U[-0.1,0.1]), odd
widths that take the scalar path, the stability and constant-row special
cases, and the reference's negative controls (uniform softmax; eps = 0).
"""
import numpy as np
import pytest

import kernelh as kh
import oracle as O
from khtest import down, empty, say, up

pytestmark = pytest.mark.gpu

SHAPES = [(4096, 1024), (16384, 4096), (1, 8192), (3, 1000), (5, 7), (64, 256), (2, 65536), (33, 2048)]


def _softmax(x, rows, cols):
    dx, dy = up(x), empty(rows * cols)
    say(f"softmax {rows}x{cols}")
    kh.softmax(dx, dy, rows, cols)
    return down(dy, rows * cols).reshape(rows, cols)


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_softmax_vs_fp64_reference(dev, rows, cols):
    x, _ = O.lcg_fill(rows * cols, 0x27AB13)
    got = _softmax(x, rows, cols)
    ref = O.ref_softmax(x, rows, cols)
    assert np.all(np.isfinite(got))
    err = np.max(np.abs(got - ref))
    print(f"softmax {rows}x{cols} max-abs={err:.3e}")
    assert err <= 1e-4


def test_softmax_bench_inputs(dev):
    rows, cols = 4096, 1024
    x = O.normal(rows * cols, 0x50F7, 0.0, 4.0)
    got = _softmax(x, rows, cols)
    assert np.max(np.abs(got - O.ref_softmax(x, rows, cols))) <= 1e-4
    assert np.max(np.abs(got.astype(np.float64).sum(axis=1) - 1.0)) <= 1e-5


def test_softmax_stability_case(dev):
    rows = cols = 1024
    pat = np.array([1000.0, -1000.0, 0.0, 0.5, -0.5], np.float32)
    x = np.tile(np.resize(pat, cols), rows)
    got = _softmax(x, rows, cols)
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - O.ref_softmax(x, rows, cols))) <= 1e-4


def test_softmax_negative_control_uniform(dev):
    rows = cols = 256
    x, _ = O.lcg_fill(rows * cols, 0x51AC0D3)
    got = _softmax(x, rows, cols)
    assert np.any(np.abs(got - 1.0 / cols) > 1e-4)


def test_softmax_reference_geometry(dev):
    rows, cols = 300, 1024
    x, _ = O.lcg_fill(rows * cols, 0x27AB13)
    dx, dy = up(x), empty(rows * cols)
    f = kh.template_function("softmax")
    args = kh.LaunchArgs().add_memref(dx, [rows, cols]).add_memref(dy, [rows, cols])
    assert args.param_count() == 14
    say("softmax reference geometry rows x 256")
    kh.kernel_launch(f, (rows, 1, 1), (256, 1, 1), args)
    assert np.max(np.abs(down(dy, rows * cols).reshape(rows, cols) - O.ref_softmax(x, rows, cols))) <= 1e-4


@pytest.mark.parametrize("symbol", ["softmax", "softmax_wide", "layernorm", "layernorm_wide"])
@pytest.mark.parametrize("cols", [64, 256, 512, 1000, 1024, 2048, 4096, 5000])
def test_every_row_symbol_at_every_width(dev, symbol, cols):
    # Each symbol of a template computes the same result at every width (the
    # launcher picks one by width; raw callers may launch either).
    rows = 37
    x, seed = O.lcg_fill(rows * cols, 0x27AB13)
    g, seed = O.lcg_fill(cols, seed)
    b, seed = O.lcg_fill(cols, seed)
    m = kh.GpuModule(kh.code_object(symbol.split("_")[0]))
    f = m.get_function(symbol)
    dx, dy = up(x), empty(rows * cols)
    args = kh.LaunchArgs().add_memref(dx, [rows, cols])
    if symbol.startswith("layernorm"):
        dg, db = up(g), up(b)
        args.add_memref(dg, [cols]).add_memref(db, [cols])
        ref = O.ref_layernorm(x, g, b, rows, cols)
    else:
        ref = O.ref_softmax(x, rows, cols)
    args.add_memref(dy, [rows, cols])
    say(f"{symbol} rows={rows} cols={cols}")
    kh.kernel_launch(f, (5, 1, 1), (256, 1, 1), args)
    got = down(dy, rows * cols).reshape(rows, cols)
    assert np.max(np.abs(got - ref)) <= 1e-4



@pytest.mark.parametrize("block", [64, 128, 192])
@pytest.mark.parametrize("cols", [128, 1024])
def test_layernorm_narrow_block_sizes(dev, block, cols):
    # The narrow symbol copies gamma and beta into LDS with the block's
    # threads before its rows: any multiple of 64 threads per block, with
    # grid-strided rows, gives the same result.
    rows = 45
    x, seed = O.lcg_fill(rows * cols, 0x51ED27)
    g, seed = O.lcg_fill(cols, seed)
    b, seed = O.lcg_fill(cols, seed)
    f = kh.GpuModule(kh.code_object("layernorm")).get_function("layernorm")
    dx, dg, db, dy = up(x), up(g), up(b), empty(rows * cols)
    args = kh.LaunchArgs().add_memref(dx, [rows, cols]).add_memref(dg, [cols]).add_memref(db, [cols])
    args.add_memref(dy, [rows, cols])
    say(f"layernorm block={block} rows={rows} cols={cols}")
    kh.kernel_launch(f, (4, 1, 1), (block, 1, 1), args)
    got = down(dy, rows * cols).reshape(rows, cols)
    assert np.max(np.abs(got - O.ref_layernorm(x, g, b, rows, cols))) <= 1e-4

def _layernorm(x, g, b, rows, cols):
    dx, dg, db, dy = up(x), up(g), up(b), empty(rows * cols)
    say(f"layernorm {rows}x{cols}")
    kh.layernorm(dx, dg, db, dy, rows, cols)
    return down(dy, rows * cols).reshape(rows, cols)


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_layernorm_vs_fp64_reference(dev, rows, cols):
    x, seed = O.lcg_fill(rows * cols, 0x2E2E8A)
    g, seed = O.lcg_fill(cols, seed)
    b, seed = O.lcg_fill(cols, seed)
    got = _layernorm(x, g, b, rows, cols)
    err = np.max(np.abs(got - O.ref_layernorm(x, g, b, rows, cols)))
    print(f"layernorm {rows}x{cols} max-abs={err:.3e}")
    assert err <= 1e-4


def test_layernorm_bench_inputs(dev):
    rows, cols = 4096, 1024
    x = O.normal(rows * cols, 0x1A7E, 0.0, 4.0)
    g = O.uniform(cols, 0x1A7F, 0.5, 1.5)
    b = O.uniform(cols, 0x1A80, -0.1, 0.1)
    got = _layernorm(x, g, b, rows, cols)
    assert np.max(np.abs(got - O.ref_layernorm(x, g, b, rows, cols))) <= 1e-4


def test_layernorm_constant_rows_and_eps0_control(dev):
    rows, cols = 64, 1024
    x = np.full(rows * cols, 3.0, np.float32)
    g, seed = O.lcg_fill(cols, 0xC0578A)
    b, seed = O.lcg_fill(cols, seed)
    got = _layernorm(x, g, b, rows, cols)
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - O.ref_layernorm(x, g, b, rows, cols))) <= 1e-4
    # Negative control (e2e_layernorm_test.cpp:336-425): the eps = 0 reference
    # is NaN everywhere, the kernel's eps = 1e-5 output is finite beta.
    ref0 = O.ref_layernorm(x, g, b, rows, cols, eps=0.0)
    assert np.all(np.isnan(ref0)) and not np.any(np.abs(got - ref0) <= 1e-4)


@pytest.mark.parametrize("template", ["softmax", "layernorm"])
@pytest.mark.parametrize("cols", [100, 40, 200])
def test_rows_blocks_of_partial_waves(dev, template, cols):
    # The reference's rows x min(cols, 256) geometry (kernelh_backend.cpp:
    # 256-257) with cols < 256 not a multiple of 64: blocks of `cols`
    # threads. The verified launch refuses them, as the reference's launch
    # verifier does; a raw launch (plain hipModuleLaunchKernel) is still
    # correct: the kernels give each thread whole rows when the block is not
    # whole wavefronts.
    rows = 70
    x, seed = O.lcg_fill(rows * cols, 0x51ED27)
    g, seed = O.lcg_fill(cols, seed)
    b, seed = O.lcg_fill(cols, seed)
    dx, dy = up(x), empty(rows * cols)
    args = kh.LaunchArgs().add_memref(dx, [rows, cols])
    if template == "layernorm":
        dg, db = up(g), up(b)
        args.add_memref(dg, [cols]).add_memref(db, [cols])
        ref = O.ref_layernorm(x, g, b, rows, cols)
    else:
        ref = O.ref_softmax(x, rows, cols)
    args.add_memref(dy, [rows, cols])
    say(f"{template} partial-wave blocks rows={rows} cols={cols} block={min(cols, 256)}")
    f = kh.template_function(template)
    with pytest.raises(kh.KhrtError, match="multiple of the wavefront size"):
        kh.kernel_launch(f, (rows, 1, 1), (min(cols, 256), 1, 1), args)
    kh.launch_raw(f, (rows, 1, 1), (min(cols, 256), 1, 1), args)
    kh.synchronize()
    got = down(dy, rows * cols).reshape(rows, cols)
    assert np.max(np.abs(got - ref)) <= 1e-4
