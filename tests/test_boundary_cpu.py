"""Host-side boundary of the khrt C-ABI, no GPU needed.

Mirrors the reference's CPU unit tests for the same pieces:
  descriptor packing   test/unit/runtime_descriptor_test.cpp:22-117
  device limits        test/unit/device_limits_test.cpp:157-216
  launch verifier      test/unit/launch_verifier_test.cpp:165-259
  occupancy            test/unit/occupancy_test.cpp:160-300
plus the C-ABI itself: libkhrt.so loads and exports every symbol that
include/khrt.h declares, and the embedded code objects are gfx950 wave64
ELF objects carrying each template's kernel symbol with the reference's
kernel-parameter count (2N+3 slots per memref).
"""
import ctypes
import os
import re
import struct
import subprocess
import sys

import numpy as np
import pytest

import kernelh as kh

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# ------------------------------------------------------------------ C-ABI exports

def _declared_functions():
    text = open(os.path.join(REPO, "include", "khrt.h")).read()
    return re.findall(r"KHRT_API\s+[\w\s\*]+?\b(\w+)\s*\(", text)


def test_library_exports_every_declared_symbol():
    names = _declared_functions()
    assert len(names) >= 45
    L = ctypes.CDLL(kh.LIB_PATH)
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"declared in include/khrt.h but not exported: {missing}"
    # And the Python binding covers each of them.
    assert set(names) <= set(kh.SIGNATURES), set(names) - set(kh.SIGNATURES)


def test_error_strings_and_version():
    assert kh.lib.khrt_error_string(kh.KHRT_E_REFUSED).decode().startswith("launch refused")
    assert kh.lib.khrt_error_string(kh.KHRT_E_SKIP).decode() == "skipped"
    assert b"gfx950" in kh.lib.khrt_version()


# ------------------------------------------------------------------ descriptors

def test_descriptor_1d_byte_layout():
    a = kh.LaunchArgs().add_memref(0x12340000, [1024])
    assert a.slots == [0x12340000, 0x12340000, 0, 1024, 1]


def test_descriptor_2d_byte_layout():
    a = kh.LaunchArgs().add_memref(0x00AABBCC, [16, 8])
    assert a.slots == [0x00AABBCC, 0x00AABBCC, 0, 16, 8, 8, 1]


def test_descriptor_4d_layout_attention():
    a = kh.LaunchArgs().add_memref(0x1000, [4, 16, 1024, 64])
    assert a.slots == [0x1000, 0x1000, 0, 4, 16, 1024, 64, 16 * 1024 * 64, 1024 * 64, 64, 1]


def test_descriptor_scalars_after_descriptors():
    a = kh.LaunchArgs().add_memref(0x1000, [256])
    a.add_scalar_bytes(struct.pack("<i", 42)).add_scalar_bytes(struct.pack("<d", 3.5))
    assert a.param_count() == 7
    assert a.slots[5] == 42
    assert a.slots[6] == 0x400C000000000000


def test_descriptor_pair_10_params_and_param_pointers():
    a = kh.LaunchArgs().add_memref(0x1000, [4096]).add_memref(0x2000, [4096])
    assert a.slots == [0x1000, 0x1000, 0, 4096, 1, 0x2000, 0x2000, 0, 4096, 1]
    arr, store = a.params()
    base = ctypes.addressof(store)
    assert [arr[i] for i in range(10)] == [base + 8 * i for i in range(10)]


@pytest.mark.parametrize("name,ranks,count", [
    ("vecadd", [1, 1, 1], 15), ("fused_gelu", [1, 1, 1], 15), ("softmax", [2, 2], 14),
    ("layernorm", [2, 1, 1, 2], 24), ("scan", [1] * 5, 25), ("scan_totals", [1] * 7, 35),
    ("gemm", [2, 2, 2], 21), ("attention", [4, 4, 4, 4], 44)])
def test_reference_parameter_counts(name, ranks, count):
    # The 2N+3 slot counts the reference's e2e tests assert
    # (e.g. e2e_scan_test.cpp:145, 158; e2e_softmax_test.cpp:153).
    assert sum(kh.lib.khrt_memref_slot_count(r) for r in ranks) == count


def test_pack_memref_capacity_error():
    buf = (ctypes.c_uint64 * 4)()
    shp = (ctypes.c_int64 * 1)(8)
    rc = kh.lib.khrt_pack_memref(buf, 4, 0x10, 1, shp)
    assert rc == kh.KHRT_E_INVALID and "capacity" in kh.last_error()


# ------------------------------------------------------------------ device limits

def test_gfx950_limits_exact_values():
    l = kh.device_limits_for("gfx950")
    assert l.lds_bytes_per_workgroup == 163840
    assert l.wavefront_size == 64
    assert l.max_threads_per_workgroup == 1024
    assert list(l.max_grid_dim) == [2147483647, 65535, 65535]
    assert l.waves_per_cu == 32
    assert l.reg_file_per_cu == 131072
    assert l.cu_count == 0
    assert l.name == b"AMD Instinct MI355X (gfx950)"


def test_reference_entries_kept():
    g = kh.device_limits_for("gfx1101")
    assert (g.lds_bytes_per_workgroup, g.wavefront_size, g.waves_per_cu, g.reg_file_per_cu) == (65536, 32, 32, 6144)
    s = kh.device_limits_for("sm_80")
    assert (s.lds_bytes_per_workgroup, s.waves_per_cu, s.reg_file_per_cu) == (49152, 64, 65536)


@pytest.mark.parametrize("bad", ["gfx90a", "", "GFX950", None])
def test_unknown_target_lists_known_tokens(bad):
    with pytest.raises(kh.KhrtError) as e:
        kh.device_limits_for(bad)
    assert e.value.code == kh.KHRT_E_UNKNOWN_TARGET
    assert "known targets: gfx950, gfx1101, sm_80" in e.value.message
    assert (f'"{bad}"' if bad is not None else '"(null)"') in e.value.message


def test_query_cu_count_falls_back_to_table_without_device():
    if kh.device_count() > 0:
        pytest.skip("a device is visible; the fallback path is for device-less hosts")
    l = kh.device_limits_for("gfx950")
    assert kh.lib.khrt_query_cu_count(ctypes.byref(l)) == 0


# ------------------------------------------------------------------ launch verifier

def test_verifier_shared_over_lds():
    d = kh.verify_launch(256, (1, 1, 1), 170000)
    assert "shared memory 170000 bytes exceeds the 163840-byte LDS limit" in d
    assert "AMD Instinct MI355X (gfx950)" in d


def test_verifier_threads_over_max():
    assert "threads per workgroup 2048 exceeds the max 1024" in kh.verify_launch(2048)


def test_verifier_wave64_multiple():
    # wave32-sized workgroups that the reference accepted on gfx1101 are
    # refused on gfx950 (launch_verifier.cpp:135-143 with wavefront 64).
    assert "threads per workgroup 96 is not a multiple of the wavefront size 64" in kh.verify_launch(96)
    assert kh.verify_launch(96, limits=kh.device_limits_for("gfx1101")) == ""


def test_verifier_grid_over_limit():
    assert "grid dim (1,1,70000) exceeds the target grid limits" in kh.verify_launch(256, (1, 1, 70000))


def test_verifier_occupancy_zero_analytic():
    low = kh.device_limits_for("gfx950")
    low.waves_per_cu = 2
    d = kh.verify_launch(256, limits=low)
    assert "occupancy would be 0 on target 'AMD Instinct MI355X (gfx950)'" in d
    assert "needs 4 wavefronts" in d
    assert kh.verify_launch(128, limits=low) == ""


def test_verifier_all_rules_reported_one_per_line():
    d = kh.verify_launch(4100, (1, 1, 70000), 170000)
    lines = d.split("\n")
    assert len(lines) == 5
    assert "shared memory" in lines[0] and "exceeds the max 1024" in lines[1]
    assert "not a multiple of the wavefront size 64" in lines[2]
    assert "grid dim" in lines[3] and "occupancy would be 0" in lines[4]


def test_verifier_accepts_template_launches():
    for name, shape in [("vecadd", "n=16777216"), ("softmax", "rows=4096,cols=1024"),
                        ("layernorm", "rows=4096,cols=1024"), ("scan", "n=67108864"),
                        ("fused_gelu", "n=67108864"), ("gemm", "m=8192,n=8192,k=8192"),
                        ("attention", "batch=4,heads=16,seq=4096,head_dim=64")]:
        grid, block = kh.geometry(name, shape)
        res = kh.resources(name) if name not in ("gemm", "attention") else {"lds_bytes": 0}
        assert kh.verify_launch(block[0] * block[1] * block[2], grid, res["lds_bytes"]) == "", name


# ------------------------------------------------------------------ occupancy

@pytest.mark.parametrize("vgpr,lds,threads,exp", [
    # (vgpr_waves, lds_blocks, thread_blocks, achieved, limiter, pct) on gfx1101,
    # the reference's hand computations (occupancy_test.cpp:160-235).
    (32, 16384, 256, (6, 4, 4, 4, 2, 12.5)),
    (64, 32768, 128, (3, 2, 8, 2, 2, 6.25)),
    (48, 8192, 512, (4, 8, 2, 2, 3, 6.25)),
    (128, 8192, 128, (1, 8, 8, 1, 1, 3.125)),
    (64, 65536, 256, (3, 1, 4, 1, 2, 3.125)),
    (0, 16384, 256, (0, 4, 4, 4, 2, 12.5)),
])
def test_occupancy_reference_hand_computations(vgpr, lds, threads, exp):
    r = kh.occupancy(vgpr, lds, threads, limits=kh.device_limits_for("gfx1101"))
    assert (r.vgpr_limited_waves, r.lds_limited_blocks, r.thread_limited_blocks, r.achieved_waves,
            r.limiter) == exp[:5]
    assert r.theoretical_pct == pytest.approx(exp[5])


@pytest.mark.parametrize("vgpr,lds,threads,exp", [
    # gfx950: R = 131072, wave 64, waves_per_cu 32, LDS 163840, 1024 threads.
    (128, 32768, 256, (16, 5, 4, 4, 3, 12.5)),    # 131072/(128*64)=16; 163840/32768=5; 1024/256=4
    (256, 65536, 256, (8, 2, 4, 2, 2, 6.25)),     # LDS-limited
    (512, 0, 64, (4, 0, 16, 4, 1, 12.5)),         # VGPR-limited, no LDS
    (8, 0, 64, (32, 0, 16, 16, 3, 50.0)),         # 256 waves capped at 32; thread bound 16
])
def test_occupancy_gfx950_hand_computations(vgpr, lds, threads, exp):
    r = kh.occupancy(vgpr, lds, threads)
    assert (r.vgpr_limited_waves, r.lds_limited_blocks, r.thread_limited_blocks, r.achieved_waves,
            r.limiter) == exp[:5]
    assert r.theoretical_pct == pytest.approx(exp[5])
    assert r.measured_blocks == -1 and b"analytic only" in r.measured_note


# ------------------------------------------------------------------ templates & code objects

def test_registry_names_and_unknown_kernel():
    assert kh.template_names() == list(kh.TEMPLATES)
    with pytest.raises(kh.KhrtError) as e:
        kh.code_object("matmul")
    assert "registered kernels: vecadd, gemm, softmax, layernorm, scan, scan_totals, fused_gelu, attention" \
        in e.value.message


@pytest.mark.parametrize("name", ["vecadd", "fused_gelu", "softmax", "layernorm", "scan", "scan_totals"])
def test_code_objects_are_gfx950_wave64_elf(name):
    blob = kh.code_object(name)
    assert blob[:4] == b"\x7fELF"
    assert struct.unpack_from("<H", blob, 18)[0] == 0xE0  # EM_AMDGPU
    assert b"gfx950" in blob
    assert name.encode() + b".kd" in blob  # the kernel descriptor symbol
    r = kh.resources(name)
    assert r["wavefront_size"] == 64
    assert r["private_segment_bytes"] == 0  # no scratch spills
    assert r["max_flat_workgroup_size"] >= 256


@pytest.mark.parametrize("name,nslots", [("vecadd", 15), ("fused_gelu", 15), ("softmax", 14),
                                         ("layernorm", 24), ("scan", 25), ("scan_totals", 35)])
def test_kernarg_segment_is_2n_plus_3_slots(name, nslots):
    import json
    co = {"scan_totals": "scan"}.get(name, name)
    notes = json.load(open(os.path.join(kh.CO_DIR, co + ".notes.json")))
    k = [x for x in notes if x["name"] == name][0]
    # Every explicit parameter is one 8-byte slot, nslots of them.
    assert k["explicit_args"] == [8] * nslots


@pytest.mark.parametrize("name,shape,grid,block", [
    ("vecadd", "n=16777216", (4096, 1, 1), (256, 1, 1)),
    ("vecadd", "n=1", (1, 1, 1), (256, 1, 1)),
    ("fused_gelu", "rows=4096,cols=1024", (1024, 1, 1), (256, 1, 1)),
    ("softmax", "rows=4096,cols=1024", (1024, 1, 1), (256, 1, 1)),
    ("layernorm", "rows=4097,cols=1024", (1025, 1, 1), (256, 1, 1)),
    ("scan", "n=1000000", (89, 1, 1), (768, 1, 1)),       # up to 1.5 * 2^20 elements: 768 threads
    ("scan", "n=1572865", (103, 1, 1), (1024, 1, 1)),
    ("scan", "n=67108864", (4370, 1, 1), (1024, 1, 1)),
    # gemm: the grid is the chosen symbol's tile count (rate x last-round fill).
    # gemm (128x256) is persistent: two workgroups per CU loop over its tiles.
    ("gemm", "m=8192,n=8192,k=8192", (512, 1, 1), (256, 1, 1)),      # 2048 tiles: 4 per workgroup
    ("gemm", "m=8192,n=8192,k=256", (512, 1, 1), (256, 1, 1)),       # skinny K
    ("gemm", "m=4096,n=4096,k=64", (512, 1, 1), (256, 1, 1)),         # exactly one round
    ("gemm", "m=12288,n=12288,k=1024", (512, 1, 1), (256, 1, 1)),    # 4608 tiles: 9 per workgroup
    ("gemm", "m=8192,n=1024,k=8192", (256, 1, 1), (512, 1, 1)),       # gemm_wide: 512 tiles of 128x128, 2 each
    ("gemm", "m=6144,n=6144,k=1024", (256, 1, 1), (512, 1, 1)),       # gemm_wide: 2304 tiles of 128x128, 9 each
    ("gemm", "m=3072,n=3072,k=3072", (512, 1, 1), (512, 1, 1)),       # 2304 tiles of 64x64 (gemm_small), 4.5 each
    ("gemm", "m=2048,n=2048,k=2048", (256, 1, 1), (512, 1, 1)),       # gemm_wide: 256 tiles of 128x128, one round
    ("gemm", "m=1024,n=1024,k=1024", (256, 1, 1), (512, 1, 1)),       # 64x64 (gemm_small), one each
    ("gemm", "m=512,n=512,k=512", (256, 1, 1), (512, 1, 1)),        # gemm_ksplit: 256 tiles of 32x32, 8 waves
    ("gemm", "m=768,n=768,k=768", (256, 1, 1), (512, 1, 1)),        # 144 tiles of 64x64: K split, 576 tiles looped
    ("gemm", "m=960,n=960,k=960", (225, 1, 1), (512, 1, 1)),        # K not a multiple of 128: 64x64
    ("gemm", "m=768,n=768,k=128", (144, 1, 1), (512, 1, 1)),        # K below 256: 64x64
    ("gemm", "m=512,n=512,k=8192", (256, 1, 1), (512, 1, 1)),       # gemm_ksplit_deep
    ("attention", "batch=4,heads=16,seq=4096,head_dim=64", (32, 16, 4), (256, 1, 1)),
])
def test_launcher_geometry(name, shape, grid, block):
    assert kh.geometry(name, shape) == (grid, block)


@pytest.mark.parametrize("name,shape,symbol", [
    ("gemm", "m=8192,n=8192,k=8192", "gemm"),
    ("gemm", "m=8192,n=8192,k=256", "gemm"),
    ("gemm", "m=8192,n=1024,k=8192", "gemm_wide"),       # outscores gemm_mid (same tile, one round per CU)
    ("gemm", "m=4096,n=2048,k=4096", "gemm_wide"),
    ("gemm", "m=4096,n=4096,k=4096", "gemm"),            # one round of 128x256 against four of 128x128
    ("gemm", "m=2560,n=2560,k=2560", "gemm_small"),      # 400 tiles of 128x128: a partial second round
    ("gemm", "m=1024,n=1024,k=1024", "gemm_small"),
    ("gemm", "m=3072,n=3072,k=3072", "gemm_small"),       # 2304 tiles of 64x64
    ("gemm", "m=2048,n=2048,k=2048", "gemm_wide"),
    ("gemm", "m=1536,n=1536,k=1536", "gemm_small"),      # 576 tiles of 64x64: more than one per CU
    ("gemm", "m=512,n=512,k=2048", "gemm_ksplit_deep"),   # 256 tiles of 32x32, deep K
    ("gemm", "m=512,n=512,k=1024", "gemm_ksplit"),
    ("gemm", "m=300,n=520,k=100", "gemm_ksplit"),
    ("gemm", "m=768,n=768,k=768", "gemm_ksplit"),            # fewer 64x64 tiles than CUs, whole 32x32 tiles
    ("gemm", "m=256,n=2048,k=2048", "gemm_ksplit_deep"),
    ("gemm", "m=1024,n=1024,k=512", "gemm_small"),           # 256 tiles of 64x64
    ("gemm", "m=760,n=768,k=768", "gemm_small"),             # an edge tile in m
    ("softmax", "rows=4096,cols=1024", "softmax"),
    ("softmax", "rows=16384,cols=4096", "softmax_wide"),
    ("layernorm", "rows=16,cols=2048", "layernorm_wide"),
    ("layernorm", "rows=16,cols=4100", "layernorm"),         # beyond the register paths: streaming
    ("scan_totals", "n=1000000", "scan_totals"),
])
def test_launch_symbol(name, shape, symbol):
    assert kh.launch_symbol(name, shape) == symbol
    # Every launch symbol has resource notes (from the code object).
    assert kh.resources(symbol)["wavefront_size"] == 64


def test_launch_symbol_errors():
    with pytest.raises(kh.KhrtError):
        kh.launch_symbol("gemm", "m=1,n=1")          # k missing
    with pytest.raises(kh.KhrtError):
        kh.launch_symbol("matmul", "n=4")
    buf = __import__("ctypes").create_string_buffer(4)
    assert kh.lib.khrt_template_launch_symbol(b"gemm", b"m=3072,n=3072,k=3072", buf, 4) != 0  # too small


@pytest.mark.parametrize("name,shape,msg", [
    ("softmax", "rows=4096", "'rows' and 'cols' are required"),
    ("attention", "batch=1,heads=1,seq=64,head_dim=32", "pinned to head_dim = 64"),
    ("gemm", "m=1,n=1,k=0", "'m', 'n' and 'k' are required and must be positive"),
    ("vecadd", "n=abc", "malformed shape"),
])
def test_geometry_errors(name, shape, msg):
    with pytest.raises(kh.KhrtError) as e:
        kh.geometry(name, shape)
    assert msg in e.value.message


def test_entry_points_validate_before_touching_a_device():
    with pytest.raises(kh.KhrtError) as e:
        kh.softmax(0x1000, 0x2000, 0, 16)
    assert "rows and cols must be positive" in e.value.message
    with pytest.raises(kh.KhrtError) as e:
        kh.vecadd(None, 0x10, 0x20, 16)
    assert "null buffer" in e.value.message
    with pytest.raises(kh.KhrtError) as e:
        kh.scan(0x1000, 0x2000, 0x3000, None, 0x5000, 1 << 20)
    assert "null buffer" in e.value.message


def test_corrupt_image_is_a_typed_error():
    with pytest.raises(kh.KhrtError) as e:
        kh.GpuModule(b"\x00" * 128)
    assert e.value.code == kh.KHRT_E_INVALID and "not an ELF" in e.value.message


@pytest.mark.parametrize("name", ["vecadd", "scan"])
def test_truncated_images_rejected_before_the_runtime(name):
    # hipModuleLoadData has no size argument, so the ELF structure is checked
    # on the host first: every truncation of a real code object is refused
    # with KHRT_E_INVALID before any HIP call (this runs without a device).
    blob = kh.code_object(name)
    for cut in list(range(64, len(blob), 97)) + [len(blob) - 1]:
        with pytest.raises(kh.KhrtError) as e:
            kh.GpuModule(blob[:cut])
        assert e.value.code == kh.KHRT_E_INVALID, (cut, e.value.message)
        assert "outside the image" in e.value.message or "truncated" in e.value.message
    bad = bytearray(blob)
    bad[18] = 0x3E  # e_machine = x86-64
    with pytest.raises(kh.KhrtError) as e:
        kh.GpuModule(bytes(bad))
    assert "not an AMDGPU code object" in e.value.message


def _elf_extent(blob: bytes):
    buf = ctypes.create_string_buffer(blob, len(blob))
    size = ctypes.c_size_t(0)
    rc = kh.lib.khrt_elf_image_size(buf, ctypes.byref(size))
    return rc, size.value


@pytest.mark.parametrize("name", ["vecadd", "fused_gelu", "softmax", "layernorm", "scan", "gemm", "attention"])
def test_elf_image_size_is_the_code_object_length(name):
    """Backend::module_load_data passes an image without its size
    (backend.hpp:75); the extent read from the ELF headers is the length
    of the code object, also with bytes after it in the caller's buffer."""
    blob = kh.code_object(name)
    assert _elf_extent(blob) == (0, len(blob))
    assert _elf_extent(blob + b"\xff" * 4096) == (0, len(blob))


def test_elf_image_size_refuses_what_is_not_a_code_object():
    blob = bytearray(kh.code_object("vecadd"))
    assert _elf_extent(b"\x00" * 128)[0] == kh.KHRT_E_INVALID
    x86 = bytearray(blob)
    x86[18] = 0x3E
    assert _elf_extent(bytes(x86))[0] == kh.KHRT_E_INVALID
    far = bytearray(blob)
    far[40:48] = struct.pack("<Q", 1 << 40)  # e_shoff far beyond any code object
    rc, _ = _elf_extent(bytes(far))
    assert rc == kh.KHRT_E_INVALID and "khrt_elf_image_size" in kh.lib.khrt_last_error().decode()


# ------------------------------------------------------------------ GEMM candidates / tune space

_PRODUCT_GEMM = ["gemm", "gemm_mid", "gemm_small", "gemm_small_pf2", "gemm_wide", "gemm_ksplit",
                 "gemm_ksplit_deep"]


def _notes(co):
    import json
    return {k["name"]: k for k in json.load(open(os.path.join(kh.CO_DIR, co + ".notes.json")))}


def test_tune_list_is_the_generators_output():
    # gemm_tune_list.h is generated by gemm_tune_space.py (which states the
    # prune rules); the committed header must be its current output.
    kdir = os.path.join(REPO, "kernel.h_amd", "csrc", "kernels")
    out = subprocess.run([sys.executable, os.path.join(kdir, "gemm_tune_space.py")], capture_output=True,
                         text=True, check=True).stdout
    assert out == open(os.path.join(kdir, "gemm_tune_list.h")).read()


def test_gemm_candidate_table():
    cands = kh.gemm_candidates()
    np_ = len(_PRODUCT_GEMM)
    assert [c["symbol"] for c in cands[:np_]] == _PRODUCT_GEMM
    assert all(c["product"] == 1 for c in cands[:np_]) and not any(c["product"] for c in cands[np_:])
    assert len({c["symbol"] for c in cands}) == len(cands)
    space = cands[np_:]
    # The reference's axes (autotuner.hpp:36-41) all vary over the space,
    # re-pruned for MFMA tiles: both MFMA shapes, 4 and 8 waves, BM/BN in
    # {64,128,256}, BK in {16,32}, unroll 1 and 2.
    assert {c["mfma"] for c in space} == {16, 32}
    assert {c["waves"] for c in space} == {4, 8}
    assert {c["bm"] for c in space} == {64, 128, 256} and {c["bn"] for c in space} == {64, 128, 256}
    assert {c["bk"] for c in space} == {16, 32}
    assert {c["unroll"] for c in space} == {1, 2}
    assert {c["pipeline"] for c in space} == {"regs", "lds-dma", "prefetch2"}
    notes = {co: _notes(co) for co in {c["code_object"] for c in cands}}
    for c in cands:
        k = notes[c["code_object"]][c["symbol"]]  # the symbol is in its code object
        assert k["max_flat_workgroup_size"] == 64 * c["waves"], c["symbol"]
        assert k["private_segment_bytes"] == 0 and k["vgpr_spill_count"] == 0, c["symbol"]
        # Two waves per SIMD: <= 256 registers; LDS for two 4-wave workgroups
        # (or one 8-wave workgroup) per CU.
        assert k["vgpr_count"] + k["agpr_count"] <= 256, c["symbol"]
        assert k["lds_bytes"] <= (160 if c["waves"] == 8 else 80) * 1024, c["symbol"]
        if not c["k_split"]:
            assert c["bm"] == c["wave_grid_m"] * c["wave_tile_m"] and c["bn"] == c["wave_grid_n"] * c["wave_tile_n"]
            assert c["wave_tile_m"] % c["mfma"] == 0 and c["wave_tile_n"] % c["mfma"] == 0
            assert c["waves"] == c["wave_grid_m"] * c["wave_grid_n"]


@pytest.mark.parametrize("symbol,m,n,k,grid,block", [
    ("gemm", 8192, 8192, 8192, 512, 256),            # persistent: two per CU
    ("gemm", 256, 512, 64, 4, 256),                  # fewer tiles than slots
    ("gemm_mid", 1000, 1000, 8, 64, 256),
    ("gemm_ksplit", 512, 512, 512, 256, 512),
    ("gemm_wide", 2048, 2048, 2048, 256, 512),      # persistent: one per CU
    ("gemm_wide", 6144, 6144, 1024, 256, 512),
    ("gemm_wide", 1000, 1000, 64, 64, 512),         # fewer tiles than CUs
    ("gemm_m16_w2x4_t4x2_k16_p1_dma", 1000, 1000, 64, 64, 512),   # 128 x 128 tiles, 8 waves
])
def test_gemm_candidate_geometry(symbol, m, n, k, grid, block):
    assert kh.gemm_candidate_geometry(symbol, m, n, k) == ((grid, 1, 1), (block, 1, 1))


def test_gemm_candidate_errors_and_tune_cache_without_device(tmp_path):
    with pytest.raises(kh.KhrtError, match="unknown GEMM candidate"):
        kh.gemm_candidate_geometry("gemm_nope", 8, 8, 8)
    c = kh.GemmCandidate()
    assert kh.lib.khrt_gemm_candidate_get(kh.lib.khrt_gemm_candidate_count(), ctypes.byref(c)) == kh.KHRT_E_INVALID
    assert "outside" in kh.last_error()
    # A cache naming a candidate changes nothing where no device gives the
    # key its device part: the built-in choice stays.
    if kh.device_count() == 0:
        p = tmp_path / "cache.json"
        p.write_text('{"key": "0000000000000000", "best": "gemm_small", "csv": ""}\n')
        kh.set_tune_cache(str(p))
        try:
            assert kh.launch_symbol("gemm", "m=8192,n=8192,k=8192") == "gemm"
        finally:
            kh.set_tune_cache(None)


# ------------------------------------------------------------------ shape text

@pytest.mark.parametrize("shape,why", [
    ("", "a dimension at offset 0"),
    ("n", "'=' after the dimension name at offset 1"),
    ("=5", "a dimension name at offset 0"),
    ("n=", "a decimal integer"),
    ("n=5,", "a dimension name at offset 4"),
    ("n=5x", "',' or the end after the integer at offset 3"),
    ("n= 5", "a decimal integer"),
    ("n=+-5", "a decimal integer"),
    ("n=99999999999999999999", "a decimal integer in int64 range"),
    ("n=4,,m=2", "a dimension name at offset 4"),
])
def test_shape_text_rejections_name_what_was_expected(shape, why):
    with pytest.raises(kh.KhrtError) as e:
        kh.geometry("vecadd", shape)
    assert "malformed shape: expected " + why in e.value.message


@pytest.mark.parametrize("shape", ["n=1024", "n=+1024", "m=1,n=1024", "n=7,n=1024"])
def test_shape_text_accepts(shape):
    """A sign, other dims, and a later dim replacing an earlier one."""
    assert kh.geometry("vecadd", shape) == kh.geometry("vecadd", "n=1024")


# ------------------------------------------------------------------ bench metrics

# Hand-computed values of test/unit/bench_metrics_test.cpp:16-83, one per
# REQUIRE, through the formulas the CLI's rate column uses.
@pytest.mark.parametrize("formula,args,value", [
    ("gflops_from_ms", (1073741824.0, 1.0), 1073.741824),
    ("gflops_from_ms", (1e9, 1.0), 1000.0),
    ("gflops_from_ms", (68719476736.0, 2.0), 34359.738368),
    ("gbps_from_ms", (3.0 * (1 << 30), 6.0), 536.870912),
    ("gemm_flops", (512, 512, 512), 268435456.0),
    ("gemm_flops", (1024, 1024, 1024), 2147483648.0),
    ("gemm_bytes", (512, 512, 512), 3145728.0),
    ("elementwise_bytes", (4096, 1024), 33554432.0),
    ("layernorm_bytes", (4096, 1024), 33562624.0),
    ("scan_bytes", (100000,), 800000.0),
    ("fused_gelu_bytes", (1048576,), 12582912.0),
    ("attention_flops", (2, 8, 512, 64), 1073741824.0),
    ("roofline_triad_bytes", (1 << 28,), 3221225472.0),
    ("roofline_fma_flops", (1 << 35,), 68719476736.0),
])
def test_bench_metric_formulas_match_the_reference_pins(formula, args, value):
    assert kh.bench_metric(formula, *args) == pytest.approx(value, rel=1e-12)


def test_bench_metric_end_to_end_gemm_rate():
    # 512^3 in 0.25 ms = 1073.741824 GFLOP/s (bench_metrics_test.cpp:78-83).
    assert kh.bench_metric("gflops_from_ms", kh.bench_metric("gemm_flops", 512, 512, 512), 0.25) == \
        pytest.approx(1073.741824, rel=1e-12)


def test_bench_metric_errors():
    with pytest.raises(kh.KhrtError, match="unknown formula"):
        kh.bench_metric("vecadd_bytes", 1.0)
    with pytest.raises(kh.KhrtError, match="takes 3 arguments, got 2"):
        kh.bench_metric("gemm_flops", 1.0, 2.0)


# Every kernelh row of the CLI's suites: its work is the reference formula
# of its kernel at its shape (fused_gelu's 12 B per element counts the dead
# tmp stream; layernorm adds 8 B per column for gamma and beta).
@pytest.mark.parametrize("kernel,shape,value,flops", [
    ("vecadd", "n=16777216", 12.0 * 16777216, False),
    ("softmax", "rows=4096,cols=1024", 33554432.0, False),
    ("layernorm", "rows=4096,cols=1024", 33562624.0, False),
    ("layernorm", "rows=16384,cols=4096", 8.0 * 16384 * 4096 + 8.0 * 4096, False),
    ("scan", "n=1000000", 8.0e6, False),
    ("fused_gelu", "n=4194304", 12.0 * 4194304, False),
    ("fused_gelu", "rows=64,cols=1024", 12.0 * 65536, False),
    ("gemm", "m=8192,n=8192,k=256", 2.0 * 8192 * 8192 * 256, True),
    ("attention", "batch=4,heads=16,seq=4096,head_dim=64", 4.0 * 4 * 16 * 4096 * 4096 * 64, True),
    ("attention", "batch=2,heads=8,seq=512", 1073741824.0, True),
    ("roofline_triad", "n=268435456", 3221225472.0, False),
])
def test_bench_row_work(kernel, shape, value, flops):
    assert kh.bench_row_work(kernel, shape) == (pytest.approx(value, rel=1e-12), flops)


def test_bench_row_work_needs_the_kernels_dims():
    with pytest.raises(kh.KhrtError, match="no bench row for kernel 'softmax'"):
        kh.bench_row_work("softmax", "n=1024")
