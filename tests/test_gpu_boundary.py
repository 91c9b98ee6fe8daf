"""GPU half of the boundary: live device limits, module loading through
hipModuleLoadData, the verified launch refusing bad configs, the occupancy
API, and the reference's raw launch protocol (caller-owned geometry,
KernelLaunch-style parameter packing) on the embedded code objects."""
import numpy as np
import pytest

import kernelh as kh
import oracle as O
from khtest import down, empty, say, up

pytestmark = pytest.mark.gpu


def test_live_device_is_gfx950(dev):
    assert dev["arch"].startswith("gfx950"), dev["arch"]
    assert dev["wavefront_size"] == 64
    assert dev["lds_bytes_per_workgroup"] == 163840
    lim = kh.live_limits()
    assert lim.cu_count == dev["cu_count"] > 0
    assert lim.lds_bytes_per_workgroup == 163840 and lim.wavefront_size == 64


@pytest.mark.parametrize("name", ["vecadd", "fused_gelu", "softmax", "layernorm", "scan", "scan_totals"])
def test_embedded_code_objects_load_and_resolve(dev, name):
    say(f"module load {name}")
    m = kh.GpuModule(kh.code_object(name))
    assert m.get_function(name)
    with pytest.raises(kh.KhrtError):
        m.get_function("no_such_kernel")
    m.unload()


def test_truncated_image_is_a_typed_error(dev):
    blob = kh.code_object("vecadd")
    with pytest.raises(kh.KhrtError) as e:
        kh.GpuModule(blob[:200])
    assert e.value.code != 0 and e.value.message


def test_verified_launch_refuses_and_never_launches(dev):
    f = kh.template_function("vecadd")
    a = kh.LaunchArgs()
    for _ in range(3):
        a.add_memref(0, [16])
    with pytest.raises(kh.KhrtError) as e:
        kh.kernel_launch(f, (1, 1, 1), (96, 1, 1), a)  # not a wave64 multiple
    assert e.value.code == kh.KHRT_E_REFUSED
    assert e.value.message.startswith("KernelLaunch::launch refused: ")
    assert "not a multiple of the wavefront size 64" in e.value.message
    with pytest.raises(kh.KhrtError) as e:
        kh.kernel_launch(f, (1, 1, 1), (256, 1, 1), kh.LaunchArgs())
    assert "no kernel arguments packed" in e.value.message


def test_measured_occupancy_api(dev):
    f = kh.template_function("softmax")
    r = kh.resources("softmax")
    rep = kh.occupancy(r["vgpr_count"], r["lds_bytes"], 256, limits=kh.live_limits(), function=f)
    assert rep.measured_blocks >= 1, rep.measured_note
    assert 0 < rep.measured_pct <= 100


def test_reference_raw_protocol_vecadd(dev):
    # The reference's e2e protocol: caller-owned geometry ceil(n/256) x 256,
    # 3 rank-1 descriptors = 15 params (e2e_vecadd_test.cpp:90-99), through
    # the verified KernelLaunch path.
    n = 65536 + 3
    a, b = O.vecadd_inputs(n)
    da, db, dc = up(a), up(b), empty(n)
    m = kh.GpuModule(kh.code_object("vecadd"))  # kept alive while f is used
    f = m.get_function("vecadd")
    args = kh.LaunchArgs().add_memref(da, [n]).add_memref(db, [n]).add_memref(dc, [n])
    assert args.param_count() == 15
    say("raw vecadd reference geometry")
    kh.kernel_launch(f, ((n + 255) // 256, 1, 1), (256, 1, 1), args)
    assert np.array_equal(down(dc, n), O.ref_vecadd(a, b))


def test_module_outlives_caller_image_buffer(dev):
    # The runtime copies the image: the caller's buffer may be freed and
    # overwritten right after the load (regression test for a freed image
    # being read by the HIP runtime after hipModuleLoadData).
    import ctypes
    blob = kh.code_object("vecadd")
    buf = ctypes.create_string_buffer(blob, len(blob))
    h = ctypes.c_void_p()
    kh.check(kh.lib.khrt_module_load_data(ctypes.byref(h), ctypes.addressof(buf), len(blob)))
    ctypes.memset(buf, 0xAB, len(blob))
    del buf
    f = ctypes.c_void_p()
    kh.check(kh.lib.khrt_module_get_function(ctypes.byref(f), h, b"vecadd"))
    n = 4096
    a, b = O.vecadd_inputs(n)
    da, db, dc = up(a), up(b), empty(n)
    args = kh.LaunchArgs().add_memref(da, [n]).add_memref(db, [n]).add_memref(dc, [n])
    say("vecadd from a module whose caller image was overwritten")
    kh.kernel_launch(f.value, (16, 1, 1), (256, 1, 1), args)
    assert np.array_equal(down(dc, n), O.ref_vecadd(a, b))
    kh.check(kh.lib.khrt_module_unload(h))


def test_function_handle_keeps_its_module_loaded(dev):
    # A handle taken from a temporary GpuModule holds the module: the module
    # is unloaded only once no handle of it is reachable (regression test
    # for a launch through the handle of a module already unloaded).
    import gc
    f = kh.GpuModule(kh.code_object("vecadd")).get_function("vecadd")
    gc.collect()
    n = 4096
    a, b = O.vecadd_inputs(n)
    da, db, dc = up(a), up(b), empty(n)
    args = kh.LaunchArgs().add_memref(da, [n]).add_memref(db, [n]).add_memref(dc, [n])
    say("vecadd through the handle of a temporary module")
    kh.kernel_launch(f, (16, 1, 1), (256, 1, 1), args)
    assert np.array_equal(down(dc, n), O.ref_vecadd(a, b))
    assert int(f) == f and f.module.handle


def test_events_time_a_launch(dev):
    n = 1 << 20
    a = up(np.ones(n, np.float32))
    c = empty(n)
    s = kh.Stream()
    e0, e1 = kh.Event(), kh.Event()
    say("event timing")
    e0.record(s)
    kh.vecadd(a, a, c, n, s)
    e1.record(s)
    e1.synchronize()
    assert 0.0 < e0.elapsed_ms(e1) < 1000.0
    assert np.all(down(c, n) == 2.0)
    s.destroy()
