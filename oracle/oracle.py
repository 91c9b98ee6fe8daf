"""ctypes/numpy front end of the CPU oracle (oracle/oracle.c).

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker (or the timed CPU
baseline), never as the product path.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None
# Builds of the same source for wider vector ISAs (oracle/Makefile).
_ISA_LIBS = {"x86-64-v2": "liboracle.so", "x86-64-v3": "liboracle_v3.so", "x86-64-v4": "liboracle_v4.so"}

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")


def build() -> None:
    """Compile liboracle.so from oracle.c (always recompiles)."""
    subprocess.run(["make", "-B", "-s", "-C", _HERE], check=True)


def host_isa() -> str:
    """The widest x86-64 level this host's CPU flags support (v4: AVX-512
    F/BW/CD/DQ/VL; v3: AVX2 + FMA + BMI2 + MOVBE), as the CPU baseline's
    stand-in for -march=native on a host the oracle was not built on."""
    flags = set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    break
    except OSError:
        return "x86-64-v2"
    if {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= flags:
        return "x86-64-v4"
    if {"avx2", "fma", "bmi2", "movbe"} <= flags:
        return "x86-64-v3"
    return "x86-64-v2"


def use_isa(level: str) -> str:
    """Loads the oracle build for x86-64 level `level` (must not exceed the
    host's, see host_isa) in place of the portable one; returns the path."""
    global _LIB_PATH, _lib
    _LIB_PATH = os.path.join(_HERE, "_build", _ISA_LIBS[level])
    _lib = None
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        c = ctypes
        sigs = {
            "kho_set_threads": (None, [c.c_int]),
            "kho_get_threads": (c.c_int, []),
            "kho_openmp_enabled": (c.c_int, []),
            "kho_lcg_fill": (None, [_f32p, c.c_size_t, c.POINTER(c.c_uint32)]),
            "kho_mt19937_raw": (None, [c.c_uint32, _u32p, c.c_size_t]),
            "kho_mt19937_fill": (None, [_f32p, c.c_size_t, c.c_uint32]),
            "kho_splitmix64_next": (c.c_uint64, [c.POINTER(c.c_uint64)]),
            "kho_fill_uniform": (None, [_f32p, c.c_size_t, c.c_uint64, c.c_double, c.c_double]),
            "kho_fill_normal": (None, [_f32p, c.c_size_t, c.c_uint64, c.c_double, c.c_double]),
            "kho_fill_vecadd": (None, [_f32p, _f32p, c.c_size_t]),
            "kho_fill_gemm_int": (None, [_f32p, _f32p, c.c_long, c.c_long, c.c_long]),
            "kho_ref_vecadd": (None, [_f32p, _f32p, _f32p, c.c_size_t]),
            "kho_ref_softmax": (None, [_f32p, _f64p, c.c_long, c.c_long, c.c_long]),
            "kho_ref_layernorm": (None, [_f32p, _f32p, _f32p, c.c_double, _f64p, c.c_long, c.c_long, c.c_long]),
            "kho_ref_scan": (None, [_f32p, _f32p, c.c_size_t, c.c_int]),
            "kho_ref_scan_exact": (None, [_f32p, _f32p, c.c_size_t, c.c_void_p, c.c_void_p]),
            "kho_ref_gelu": (None, [_f32p, _f64p, c.c_size_t, c.c_int]),
            "kho_ref_gemm": (None, [_f32p, _f32p, _f64p, c.c_long, c.c_long, c.c_long, c.c_long, c.c_long, c.c_int]),
            "kho_ref_attention_rows": (None, [_f32p, _f32p, _f32p, _f64p, c.c_long, c.c_long, c.c_int, _i64p, _i64p, c.c_long]),
            "kho_emu_softmax": (None, [_f32p, _f32p, c.c_long, c.c_long]),
            "kho_emu_layernorm": (None, [_f32p, _f32p, _f32p, _f32p, c.c_long, c.c_long]),
            "kho_emu_gelu": (None, [_f32p, _f32p, c.c_size_t]),
            "kho_emu_scan_template": (None, [_f32p, _f32p, c.c_size_t]),
            "kho_emu_gemm": (None, [_f32p, _f32p, _f32p, c.c_long, c.c_long, c.c_long, c.c_long]),
            "kho_emu_attention_rows": (None, [_f32p, _f32p, _f32p, _f32p, c.c_long, c.c_long, _i64p, _i64p, c.c_long]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def set_threads(n: int) -> None:
    lib().kho_set_threads(int(n))


# ---------------------------------------------------------------- generators

def lcg_fill(n: int, seed: int) -> tuple[np.ndarray, int]:
    """LCG fill of n floats; returns (values, next seed)."""
    v = np.empty(n, np.float32)
    s = ctypes.c_uint32(seed)
    lib().kho_lcg_fill(v, n, ctypes.byref(s))
    return v, s.value


def mt19937_raw(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().kho_mt19937_raw(seed, out, n)
    return out


def mt19937_fill(n: int, seed: int) -> np.ndarray:
    v = np.empty(n, np.float32)
    lib().kho_mt19937_fill(v, n, seed)
    return v


def splitmix64(state: int, count: int) -> list[int]:
    st = ctypes.c_uint64(state)
    return [lib().kho_splitmix64_next(ctypes.byref(st)) for _ in range(count)]


def uniform(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    v = np.empty(n, np.float32)
    lib().kho_fill_uniform(v, n, seed, lo, hi)
    return v


def normal(n: int, seed: int, mean: float, sd: float) -> np.ndarray:
    v = np.empty(n, np.float32)
    lib().kho_fill_normal(v, n, seed, mean, sd)
    return v


def vecadd_inputs(n: int) -> tuple[np.ndarray, np.ndarray]:
    a = np.empty(n, np.float32)
    b = np.empty(n, np.float32)
    lib().kho_fill_vecadd(a, b, n)
    return a, b


def gemm_int_inputs(m: int, n: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    A = np.empty(m * k, np.float32)
    B = np.empty(k * n, np.float32)
    lib().kho_fill_gemm_int(A, B, m, n, k)
    return A.reshape(m, k), B.reshape(k, n)


# ---------------------------------------------------------------- references

def _c32(x):
    return np.ascontiguousarray(x, dtype=np.float32).reshape(-1)


def ref_vecadd(a, b) -> np.ndarray:
    a, b = _c32(a), _c32(b)
    c = np.empty_like(a)
    lib().kho_ref_vecadd(a, b, c, a.size)
    return c


def ref_softmax(x, rows: int, cols: int, row0: int = 0, nrows: int | None = None) -> np.ndarray:
    nrows = rows - row0 if nrows is None else nrows
    y = np.empty(nrows * cols, np.float64)
    lib().kho_ref_softmax(_c32(x), y, cols, row0, nrows)
    return y.reshape(nrows, cols)


def ref_layernorm(x, gamma, beta, rows: int, cols: int, eps: float = 1e-5, row0: int = 0,
                  nrows: int | None = None) -> np.ndarray:
    nrows = rows - row0 if nrows is None else nrows
    y = np.empty(nrows * cols, np.float64)
    lib().kho_ref_layernorm(_c32(x), _c32(gamma), _c32(beta), eps, y, cols, row0, nrows)
    return y.reshape(nrows, cols)


def ref_scan(x, exclusive: bool = False) -> np.ndarray:
    x = _c32(x)
    y = np.empty_like(x)
    lib().kho_ref_scan(x, y, x.size, 1 if exclusive else 0)
    return y


def ref_scan_exact(x, with_abs: bool = False, with_margin: bool = False):
    """Correctly rounded fp32 inclusive prefix (exact long accumulator).
    With with_abs, also returns the fp64 running sum of |x|; with
    with_margin, each prefix's distance from the nearest point where its
    fp32 rounding would change (min(spacing below, spacing above)/2 minus
    |exact - rounded|)."""
    x = _c32(x)
    y = np.empty_like(x)
    a = np.empty(x.size, np.float64) if with_abs else None
    m = np.empty(x.size, np.float64) if with_margin else None
    lib().kho_ref_scan_exact(x, y, x.size, a.ctypes.data if with_abs else None,
                             m.ctypes.data if with_margin else None)
    out = (y,) + ((a,) if with_abs else ()) + ((m,) if with_margin else ())
    return out if len(out) > 1 else y


def ref_gelu(x, with_tanh: bool = True) -> np.ndarray:
    x = _c32(x)
    y = np.empty(x.size, np.float64)
    lib().kho_ref_gelu(x, y, x.size, 1 if with_tanh else 0)
    return y


def ref_gemm(A, B, m: int, n: int, k: int, row0: int = 0, nrows: int | None = None,
             transpose_b: bool = False) -> np.ndarray:
    nrows = m - row0 if nrows is None else nrows
    C = np.empty(nrows * n, np.float64)
    lib().kho_ref_gemm(_c32(A), _c32(B), C, m, n, k, row0, nrows, 1 if transpose_b else 0)
    return C.reshape(nrows, n)


def ref_attention_rows(Q, K, V, seq: int, d: int, bh, qi, scaled: bool = True) -> np.ndarray:
    bh = np.ascontiguousarray(bh, dtype=np.int64)
    qi = np.ascontiguousarray(qi, dtype=np.int64)
    O = np.empty(bh.size * d, np.float64)
    lib().kho_ref_attention_rows(_c32(Q), _c32(K), _c32(V), O, seq, d, 1 if scaled else 0, bh, qi, bh.size)
    return O.reshape(bh.size, d)


# ---------------------------------------------------------------- emulators

def emu_softmax(x, rows: int, cols: int) -> np.ndarray:
    y = np.empty(rows * cols, np.float32)
    lib().kho_emu_softmax(_c32(x), y, rows, cols)
    return y.reshape(rows, cols)


def emu_layernorm(x, gamma, beta, rows: int, cols: int) -> np.ndarray:
    y = np.empty(rows * cols, np.float32)
    lib().kho_emu_layernorm(_c32(x), _c32(gamma), _c32(beta), y, rows, cols)
    return y.reshape(rows, cols)


def emu_gelu(x) -> np.ndarray:
    x = _c32(x)
    y = np.empty_like(x)
    lib().kho_emu_gelu(x, y, x.size)
    return y


def emu_scan_template(x) -> np.ndarray:
    x = _c32(x)
    y = np.empty_like(x)
    lib().kho_emu_scan_template(x, y, x.size)
    return y


def emu_gemm(A, B, m: int, n: int, k: int, row0: int = 0, nrows: int | None = None) -> np.ndarray:
    nrows = m - row0 if nrows is None else nrows
    C = np.empty(nrows * n, np.float32)
    lib().kho_emu_gemm(_c32(A), _c32(B), C, n, k, row0, nrows)
    return C.reshape(nrows, n)


def emu_attention_rows(Q, K, V, seq: int, d: int, bh, qi) -> np.ndarray:
    bh = np.ascontiguousarray(bh, dtype=np.int64)
    qi = np.ascontiguousarray(qi, dtype=np.int64)
    O = np.empty(bh.size * d, np.float32)
    lib().kho_emu_attention_rows(_c32(Q), _c32(K), _c32(V), O, seq, d, bh, qi, bh.size)
    return O.reshape(bh.size, d)


# ---------------------------------------------------------------- checks

def rel_frobenius(c, ref) -> float:
    """||c - ref||_F / ||ref||_F in fp64 (test/unit/e2e_gemm_test.cpp:113-125)."""
    c = np.asarray(c, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.sqrt(np.sum((c - ref) ** 2) / np.sum(ref ** 2)))


def attention_violation(got, ref, rtol: float = 2e-3) -> float:
    """max(|g - r| - rtol*|r|): the per-element rule |g-r| <= atol + rtol*|r|
    holds iff this is <= atol (test/unit/e2e_attention_test.cpp:298-311)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref) - rtol * np.abs(ref)))
