"""Python front end of the khrt C-ABI (include/khrt.h) via ctypes.

This is a thin binding: every call goes to libkhrt.so, which loads the
embedded gfx950 code objects with hipModuleLoadData and launches them with
hipModuleLaunchKernel. There is no Python or CPU fallback for any kernel: if
the library is missing, importing this module raises.

The classes mirror the reference runtime's C++ shapes
(include/kernelh/runtime/*.hpp): Buffer (buffer.hpp), GpuModule
(gpu_module.hpp), LaunchArgs (descriptor_packing.hpp), EventTimer
(event_timer.hpp). Errors surface as KhrtError(code, message), the
Error{code, message} pair of runtime_error.hpp.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
BUILD = os.path.join(PKG, "build")
LIB_PATH = os.path.join(BUILD, "libkhrt.so")
CLI_PATH = os.path.join(BUILD, "kernelh")
CO_DIR = os.path.join(BUILD, "co")

KHRT_OK = 0
KHRT_E_INVALID = 1
KHRT_E_REFUSED = 2
KHRT_E_UNKNOWN_TARGET = 3
KHRT_E_NO_DEVICE = 4
KHRT_E_SKIP = 77

TEMPLATES = ("vecadd", "gemm", "softmax", "layernorm", "scan", "scan_totals", "fused_gelu", "attention")


class KhrtError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class Dim3(ctypes.Structure):
    _fields_ = [("x", ctypes.c_uint), ("y", ctypes.c_uint), ("z", ctypes.c_uint)]

    def tuple(self):
        return (self.x, self.y, self.z)


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64),
                ("lds_bytes_per_workgroup", ctypes.c_int64), ("wavefront_size", ctypes.c_int32),
                ("max_threads_per_workgroup", ctypes.c_int32), ("cu_count", ctypes.c_int64),
                ("vram_bytes", ctypes.c_int64), ("max_grid_dim", ctypes.c_int64 * 3),
                ("clock_khz", ctypes.c_int32), ("memory_clock_khz", ctypes.c_int32),
                ("memory_bus_width", ctypes.c_int32), ("l2_bytes", ctypes.c_int32)]


class DeviceLimits(ctypes.Structure):
    _fields_ = [("lds_bytes_per_workgroup", ctypes.c_int64), ("wavefront_size", ctypes.c_int32),
                ("max_threads_per_workgroup", ctypes.c_int32), ("max_grid_dim", ctypes.c_int64 * 3),
                ("vram_bytes", ctypes.c_int64), ("waves_per_cu", ctypes.c_int32),
                ("reg_file_per_cu", ctypes.c_int32), ("cu_count", ctypes.c_int64), ("name", ctypes.c_char_p)]


class LaunchConfig(ctypes.Structure):
    _fields_ = [("threads_per_workgroup", ctypes.c_int32), ("grid_x", ctypes.c_int32),
                ("grid_y", ctypes.c_int32), ("grid_z", ctypes.c_int32), ("static_shared_bytes", ctypes.c_size_t)]


class OccupancyInput(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_char_p), ("target", ctypes.c_char_p), ("config", ctypes.c_char_p),
                ("vgpr_count", ctypes.c_int32), ("lds_bytes", ctypes.c_int64),
                ("threads_per_workgroup", ctypes.c_int32)]


class OccupancyReport(ctypes.Structure):
    _fields_ = [("vgpr_limited_waves", ctypes.c_int32), ("lds_limited_blocks", ctypes.c_int32),
                ("thread_limited_blocks", ctypes.c_int32), ("achieved_waves", ctypes.c_int32),
                ("theoretical_pct", ctypes.c_double), ("limiter", ctypes.c_int32),
                ("measured_blocks", ctypes.c_int32), ("measured_pct", ctypes.c_double),
                ("measured_note", ctypes.c_char * 256)]


class KernelResources(ctypes.Structure):
    _fields_ = [("vgpr_count", ctypes.c_int32), ("agpr_count", ctypes.c_int32), ("sgpr_count", ctypes.c_int32),
                ("lds_bytes", ctypes.c_int64), ("private_segment_bytes", ctypes.c_int64),
                ("wavefront_size", ctypes.c_int32), ("max_flat_workgroup_size", ctypes.c_int32)]


class GemmCandidate(ctypes.Structure):
    _fields_ = [("symbol", ctypes.c_char * 64), ("code_object", ctypes.c_char * 16),
                ("pipeline", ctypes.c_char * 16), ("mfma", ctypes.c_int32), ("waves", ctypes.c_int32),
                ("wave_grid_m", ctypes.c_int32), ("wave_grid_n", ctypes.c_int32),
                ("wave_tile_m", ctypes.c_int32), ("wave_tile_n", ctypes.c_int32),
                ("bm", ctypes.c_int32), ("bn", ctypes.c_int32), ("bk", ctypes.c_int32),
                ("unroll", ctypes.c_int32), ("prio", ctypes.c_int32), ("persistent", ctypes.c_int32),
                ("k_split", ctypes.c_int32), ("product", ctypes.c_int32)]


_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t

# name -> (restype, argtypes). Every int-returning function is a status.
SIGNATURES = {
    "khrt_last_error": (ctypes.c_char_p, []),
    "khrt_error_string": (ctypes.c_char_p, [_i]),
    "khrt_version": (ctypes.c_char_p, []),
    "khrt_device_count": (_i, [ctypes.POINTER(_i)]),
    "khrt_init_device": (_i, [_i]),
    "khrt_get_device_info": (_i, [ctypes.POINTER(DeviceInfo)]),
    "khrt_device_synchronize": (_i, []),
    "khrt_malloc": (_i, [ctypes.POINTER(_vp), _sz]),
    "khrt_free": (_i, [_vp]),
    "khrt_memcpy_h2d": (_i, [_vp, _vp, _sz]),
    "khrt_memcpy_d2h": (_i, [_vp, _vp, _sz]),
    "khrt_memcpy_d2d": (_i, [_vp, _vp, _sz]),
    "khrt_fill_f32": (_i, [_vp, ctypes.c_float, _sz, _vp]),
    "khrt_module_load_data": (_i, [ctypes.POINTER(_vp), _vp, _sz]),
    "khrt_elf_image_size": (_i, [_vp, ctypes.POINTER(_sz)]),
    "khrt_module_get_function": (_i, [ctypes.POINTER(_vp), _vp, ctypes.c_char_p]),
    "khrt_module_unload": (_i, [_vp]),
    "khrt_launch_raw": (_i, [_vp, Dim3, Dim3, _sz, _vp, ctypes.POINTER(_vp)]),
    "khrt_stream_create": (_i, [ctypes.POINTER(_vp)]),
    "khrt_stream_destroy": (_i, [_vp]),
    "khrt_stream_synchronize": (_i, [_vp]),
    "khrt_event_create": (_i, [ctypes.POINTER(_vp)]),
    "khrt_event_record": (_i, [_vp, _vp]),
    "khrt_event_synchronize": (_i, [_vp]),
    "khrt_event_elapsed_ms": (_i, [ctypes.POINTER(ctypes.c_float), _vp, _vp]),
    "khrt_event_destroy": (_i, [_vp]),
    "khrt_memref_slot_count": (_sz, [_i]),
    "khrt_pack_memref": (_i, [ctypes.POINTER(ctypes.c_uint64), _sz, _vp, _i, ctypes.POINTER(_i64)]),
    "khrt_pack_scalar": (_i, [ctypes.POINTER(ctypes.c_uint64), _vp, _sz]),
    "khrt_device_limits_for": (_i, [ctypes.c_char_p, ctypes.POINTER(DeviceLimits)]),
    "khrt_device_target_count": (_i, []),
    "khrt_device_target_name": (ctypes.c_char_p, [_i]),
    "khrt_query_cu_count": (_i64, [ctypes.POINTER(DeviceLimits)]),
    "khrt_live_limits": (_i, [ctypes.POINTER(DeviceLimits)]),
    "khrt_verify_launch": (_i, [ctypes.POINTER(LaunchConfig), ctypes.POINTER(DeviceLimits), _vp,
                                ctypes.c_char_p, _sz]),
    "khrt_compute_occupancy": (_i, [ctypes.POINTER(OccupancyInput), ctypes.POINTER(DeviceLimits), _vp,
                                    ctypes.POINTER(OccupancyReport)]),
    "khrt_kernel_launch": (_i, [_vp, Dim3, Dim3, _sz, _vp, ctypes.POINTER(_vp), _sz]),
    "khrt_template_count": (_i, []),
    "khrt_template_name": (ctypes.c_char_p, [_i]),
    "khrt_template_code_object": (_i, [ctypes.c_char_p, ctypes.POINTER(_vp), ctypes.POINTER(_sz)]),
    "khrt_template_resources": (_i, [ctypes.c_char_p, ctypes.POINTER(KernelResources)]),
    "khrt_template_geometry": (_i, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(Dim3), ctypes.POINTER(Dim3)]),
    "khrt_template_launch_symbol": (_i, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]),
    "khrt_template_function": (_i, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "khrt_gemm_candidate_count": (_i, []),
    "khrt_gemm_candidate_get": (_i, [_i, ctypes.POINTER(GemmCandidate)]),
    "khrt_gemm_candidate_geometry": (_i, [ctypes.c_char_p, _i64, _i64, _i64, ctypes.POINTER(Dim3),
                                          ctypes.POINTER(Dim3)]),
    "khrt_gemm_candidate_function": (_i, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "khrt_set_tune_cache": (_i, [ctypes.c_char_p]),
    "khrt_tune_cache_key": (_i, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _sz]),
    "khrt_device_token": (_i, [ctypes.c_char_p, _sz]),
    "kh_vecadd": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "kh_fused_gelu": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "kh_softmax": (_i, [_vp, _vp, _i64, _i64, _vp]),
    "kh_layernorm": (_i, [_vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "kh_scan": (_i, [_vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "kh_scan_noalloc": (_i, [_vp, _vp, _i64, _vp]),
    "kh_scan_totals": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "kh_gemm": (_i, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "kh_attention": (_i, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "kh_roofline_triad": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "kh_roofline_copy": (_i, [_vp, _vp, _i64, _vp]),
    "kh_roofline_mfma": (_i, [_vp, _i64, _i64, _vp]),
    "khrt_bench_metric": (_i, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), _i, ctypes.POINTER(ctypes.c_double)]),
    "khrt_bench_row_work": (_i, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                 ctypes.POINTER(_i)]),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libkhrt.so not built at {LIB_PATH}: run `python kernel.h_amd/build.py` "
                          "(or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


lib = _load()


def last_error() -> str:
    return (lib.khrt_last_error() or b"").decode()


def check(rc: int) -> None:
    if rc != 0:
        raise KhrtError(rc, last_error())


def _ptr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, (Buffer, Stream, Event)):
        return x.ptr
    return int(x)


# ------------------------------------------------------------------ device

def device_count() -> int:
    c = ctypes.c_int(0)
    rc = lib.khrt_device_count(ctypes.byref(c))
    return c.value if rc == 0 else 0


def init_device(ordinal: int = 0) -> None:
    check(lib.khrt_init_device(ordinal))


def device_info() -> dict:
    d = DeviceInfo()
    check(lib.khrt_get_device_info(ctypes.byref(d)))
    return {"name": d.name.decode(), "arch": d.arch.decode(), "lds_bytes_per_workgroup": d.lds_bytes_per_workgroup,
            "wavefront_size": d.wavefront_size, "max_threads_per_workgroup": d.max_threads_per_workgroup,
            "cu_count": d.cu_count, "vram_bytes": d.vram_bytes, "max_grid_dim": list(d.max_grid_dim),
            "clock_khz": d.clock_khz, "memory_clock_khz": d.memory_clock_khz,
            "memory_bus_width": d.memory_bus_width, "l2_bytes": d.l2_bytes}


def synchronize() -> None:
    check(lib.khrt_device_synchronize())


class Buffer:
    """Device buffer (buffer.hpp): hipMalloc/hipFree + synchronous copies."""

    def __init__(self, nbytes: int):
        p = ctypes.c_void_p()
        check(lib.khrt_malloc(ctypes.byref(p), int(nbytes)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "Buffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.copy_from_host(a)
        return b

    def copy_from_host(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise KhrtError(KHRT_E_INVALID, "copy_from_host: source larger than buffer")
        check(lib.khrt_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes))

    def to_host(self, dtype=np.float32, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype)
        check(lib.khrt_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def fill(self, value: float, stream=None) -> None:
        check(lib.khrt_fill_f32(self.ptr, float(value), self.nbytes // 4, _ptr(stream)))

    def free(self) -> None:
        if self.ptr:
            check(lib.khrt_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr:
                lib.khrt_free(self.ptr)
        except Exception:
            pass


class Function(int):
    """A kernel handle from GpuModule.get_function: the integer handle the C
    ABI takes, holding a reference to its module so the module (and with it
    the handle) cannot be unloaded while the handle is still reachable, e.g.
    `GpuModule(image).get_function(name)` on a temporary module."""

    def __new__(cls, handle: int, module: "GpuModule"):
        obj = super().__new__(cls, handle)
        obj.module = module
        return obj


class GpuModule:
    """Loaded code object (gpu_module.hpp): hipModuleLoadData / GetFunction.
    The runtime keeps its own copy of the image; the module is unloaded when
    this object is (RAII, as GpuModule's destructor in the reference)."""

    def __init__(self, image: bytes):
        self.handle = None
        buf = ctypes.create_string_buffer(image, len(image))
        m = ctypes.c_void_p()
        check(lib.khrt_module_load_data(ctypes.byref(m), ctypes.addressof(buf), len(image)))
        self.handle = m.value

    def __del__(self):
        try:
            if self.handle:
                lib.khrt_module_unload(self.handle)
        except Exception:
            pass

    def get_function(self, name: str) -> Function:
        f = ctypes.c_void_p()
        check(lib.khrt_module_get_function(ctypes.byref(f), self.handle, name.encode()))
        return Function(f.value, self)

    def unload(self) -> None:
        if self.handle:
            check(lib.khrt_module_unload(self.handle))
            self.handle = None


class LaunchArgs:
    """Kernel parameter slots (descriptor_packing.hpp): 2N+3 per memref."""

    def __init__(self):
        self.slots: list[int] = []

    def add_memref(self, ptr, shape) -> "LaunchArgs":
        shape = [int(s) for s in shape]
        n = lib.khrt_memref_slot_count(len(shape))
        buf = (ctypes.c_uint64 * n)()
        shp = (ctypes.c_int64 * max(1, len(shape)))(*shape)
        check(lib.khrt_pack_memref(buf, n, _ptr(ptr) or 0, len(shape), shp))
        self.slots.extend(int(v) for v in buf)
        return self

    def add_scalar_bytes(self, raw: bytes) -> "LaunchArgs":
        slot = ctypes.c_uint64()
        tmp = ctypes.create_string_buffer(raw, len(raw))
        check(lib.khrt_pack_scalar(ctypes.byref(slot), ctypes.addressof(tmp), len(raw)))
        self.slots.append(slot.value)
        return self

    def param_count(self) -> int:
        return len(self.slots)

    def params(self):
        """(kernelParams array, backing storage); keep both alive."""
        store = (ctypes.c_uint64 * len(self.slots))(*self.slots)
        arr = (ctypes.c_void_p * len(self.slots))(
            *[ctypes.addressof(store) + 8 * i for i in range(len(self.slots))])
        return arr, store


def kernel_launch(function: int, grid, block, args: LaunchArgs, stream=None, shared: int = 0) -> None:
    """KernelLaunch::launch: verified against the live limits, then launched."""
    arr, store = args.params()
    check(lib.khrt_kernel_launch(function, Dim3(*grid), Dim3(*block), shared, _ptr(stream), arr, len(args.slots)))
    del store


def launch_raw(function: int, grid, block, args: LaunchArgs, stream=None, shared: int = 0) -> None:
    arr, store = args.params()
    check(lib.khrt_launch_raw(function, Dim3(*grid), Dim3(*block), shared, _ptr(stream), arr))
    del store


class Stream:
    def __init__(self):
        s = ctypes.c_void_p()
        check(lib.khrt_stream_create(ctypes.byref(s)))
        self.ptr = s.value

    def synchronize(self) -> None:
        check(lib.khrt_stream_synchronize(self.ptr))

    def destroy(self) -> None:
        if self.ptr:
            check(lib.khrt_stream_destroy(self.ptr))
            self.ptr = None


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(lib.khrt_event_create(ctypes.byref(e)))
        self.ptr = e.value

    def record(self, stream=None) -> None:
        check(lib.khrt_event_record(self.ptr, _ptr(stream)))

    def synchronize(self) -> None:
        check(lib.khrt_event_synchronize(self.ptr))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib.khrt_event_elapsed_ms(ctypes.byref(ms), self.ptr, end.ptr))
        return ms.value

    def destroy(self) -> None:
        if self.ptr:
            lib.khrt_event_destroy(self.ptr)
            self.ptr = None


# ------------------------------------------------------------------ limits

def device_limits_for(target: str) -> DeviceLimits:
    out = DeviceLimits()
    check(lib.khrt_device_limits_for(target.encode() if target is not None else None, ctypes.byref(out)))
    return out


def live_limits() -> DeviceLimits:
    out = DeviceLimits()
    check(lib.khrt_live_limits(ctypes.byref(out)))
    return out


def verify_launch(threads: int, grid=(1, 1, 1), shared: int = 0, limits: DeviceLimits | None = None,
                  function: int | None = None) -> str:
    """Returns "" when launchable, else the multi-line diagnostic."""
    cfg = LaunchConfig(threads, grid[0], grid[1], grid[2], shared)
    limits = limits if limits is not None else device_limits_for("gfx950")
    diag = ctypes.create_string_buffer(4096)
    rc = lib.khrt_verify_launch(ctypes.byref(cfg), ctypes.byref(limits), function, diag, 4096)
    if rc not in (0, KHRT_E_REFUSED):
        check(rc)
    return diag.value.decode()


def occupancy(vgpr: int, lds: int, threads: int, limits: DeviceLimits | None = None,
              function: int | None = None, kernel: str = "", config: str = "") -> OccupancyReport:
    inp = OccupancyInput(kernel.encode(), b"gfx950", config.encode(), vgpr, lds, threads)
    limits = limits if limits is not None else device_limits_for("gfx950")
    out = OccupancyReport()
    check(lib.khrt_compute_occupancy(ctypes.byref(inp), ctypes.byref(limits), function, ctypes.byref(out)))
    return out


# ------------------------------------------------------------------ templates

def template_names() -> list[str]:
    return [lib.khrt_template_name(i).decode() for i in range(lib.khrt_template_count())]


def code_object(name: str) -> bytes:
    p = ctypes.c_void_p()
    n = ctypes.c_size_t()
    check(lib.khrt_template_code_object(name.encode(), ctypes.byref(p), ctypes.byref(n)))
    return ctypes.string_at(p.value, n.value)


def resources(name: str) -> dict:
    r = KernelResources()
    check(lib.khrt_template_resources(name.encode(), ctypes.byref(r)))
    return {f: getattr(r, f) for f, _ in KernelResources._fields_}


def geometry(name: str, shape: str):
    g, b = Dim3(), Dim3()
    check(lib.khrt_template_geometry(name.encode(), shape.encode(), ctypes.byref(g), ctypes.byref(b)))
    return g.tuple(), b.tuple()


def launch_symbol(name: str, shape: str) -> str:
    """Kernel symbol the launcher runs for template `name` at `shape`."""
    buf = ctypes.create_string_buffer(64)
    check(lib.khrt_template_launch_symbol(name.encode(), shape.encode(), buf, 64))
    return buf.value.decode()


def template_function(name: str) -> int:
    f = ctypes.c_void_p()
    check(lib.khrt_template_function(name.encode(), ctypes.byref(f)))
    return f.value


def gemm_candidates() -> list[dict]:
    """Every GEMM candidate (launcher symbols first, then the tune space)."""
    out = []
    for i in range(lib.khrt_gemm_candidate_count()):
        c = GemmCandidate()
        check(lib.khrt_gemm_candidate_get(i, ctypes.byref(c)))
        d = {f: getattr(c, f) for f, _ in GemmCandidate._fields_}
        for f in ("symbol", "code_object", "pipeline"):
            d[f] = d[f].decode()
        out.append(d)
    return out


def gemm_candidate_geometry(symbol: str, m: int, n: int, k: int):
    g, b = Dim3(), Dim3()
    check(lib.khrt_gemm_candidate_geometry(symbol.encode(), m, n, k, ctypes.byref(g), ctypes.byref(b)))
    return g.tuple(), b.tuple()


def gemm_candidate_function(symbol: str) -> int:
    f = ctypes.c_void_p()
    check(lib.khrt_gemm_candidate_function(symbol.encode(), ctypes.byref(f)))
    return f.value


def set_tune_cache(path: str | None) -> None:
    """Points the GEMM launcher at a `kernelh tune` cache file (None: off)."""
    check(lib.khrt_set_tune_cache(path.encode() if path else None))


def tune_cache_key(kernel: str, shape: str) -> str:
    buf = ctypes.create_string_buffer(17)
    check(lib.khrt_tune_cache_key(kernel.encode(), shape.encode(), buf, 17))
    return buf.value.decode()


def device_token() -> str:
    buf = ctypes.create_string_buffer(512)
    check(lib.khrt_device_token(buf, 512))
    return buf.value.decode()


def vecadd(a, b, c, n: int, stream=None) -> None:
    check(lib.kh_vecadd(_ptr(a), _ptr(b), _ptr(c), n, _ptr(stream)))


def fused_gelu(x, tmp, out, n: int, stream=None) -> None:
    check(lib.kh_fused_gelu(_ptr(x), _ptr(tmp), _ptr(out), n, _ptr(stream)))


def softmax(x, y, rows: int, cols: int, stream=None) -> None:
    check(lib.kh_softmax(_ptr(x), _ptr(y), rows, cols, _ptr(stream)))


def layernorm(x, gamma, beta, y, rows: int, cols: int, stream=None) -> None:
    check(lib.kh_layernorm(_ptr(x), _ptr(gamma), _ptr(beta), _ptr(y), rows, cols, _ptr(stream)))


def scan(x, y, y_lo, totals_hi, totals_lo, n: int, stream=None) -> None:
    check(lib.kh_scan(_ptr(x), _ptr(y), _ptr(y_lo), _ptr(totals_hi), _ptr(totals_lo), n, _ptr(stream)))


def scan_noalloc(x, y, n: int, stream=None) -> None:
    """kh_scan without caller totals and without allocating (khrt.h)."""
    check(lib.kh_scan_noalloc(_ptr(x), _ptr(y), n, _ptr(stream)))


def scan_totals(totals_hi, totals_lo, off_hi, off_lo, off_lo2, y, y_lo, n: int, stream=None) -> None:
    check(lib.kh_scan_totals(_ptr(totals_hi), _ptr(totals_lo), _ptr(off_hi), _ptr(off_lo), _ptr(off_lo2),
                             _ptr(y), _ptr(y_lo), n, _ptr(stream)))


def gemm(A, B, C, m: int, n: int, k: int, stream=None) -> None:
    check(lib.kh_gemm(_ptr(A), _ptr(B), _ptr(C), m, n, k, _ptr(stream)))


def attention(Q, K, V, O, batch: int, heads: int, seq: int, head_dim: int, stream=None) -> None:
    check(lib.kh_attention(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), batch, heads, seq, head_dim, _ptr(stream)))


def roofline_triad(a, b, c, n: int, stream=None) -> None:
    check(lib.kh_roofline_triad(_ptr(a), _ptr(b), _ptr(c), n, _ptr(stream)))


def roofline_copy(src, dst, n: int, stream=None) -> None:
    check(lib.kh_roofline_copy(_ptr(src), _ptr(dst), n, _ptr(stream)))


def roofline_mfma(out, blocks: int, iters: int, stream=None) -> float:
    """Launches the MFMA microbenchmark; returns the FLOPs it executes."""
    check(lib.kh_roofline_mfma(_ptr(out), blocks, iters, _ptr(stream)))
    return float(blocks) * 4 * iters * 8 * 4096


def bench_metric(formula: str, *args: float) -> float:
    """One of the reference's bench metric formulas (bench/harness/metrics.cpp)."""
    a = (ctypes.c_double * max(1, len(args)))(*args)
    out = ctypes.c_double()
    check(lib.khrt_bench_metric(formula.encode(), a, len(args), ctypes.byref(out)))
    return out.value


def bench_row_work(kernel: str, shape: str) -> tuple[float, bool]:
    """(work per launch, is_flops) of a `kernelh bench` row."""
    w, f = ctypes.c_double(), _i()
    check(lib.khrt_bench_row_work(kernel.encode(), shape.encode(), ctypes.byref(w), ctypes.byref(f)))
    return w.value, bool(f.value)


def scan_workspace_floats(n: int) -> int:
    """Elements of each totals buffer: T = ceil(n / 256) (scan.cpp:190)."""
    return (n + 255) // 256
