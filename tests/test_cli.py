"""The `kernelh` CLI contract (tools/kernelh/main.cpp; test/lit/cli/compile.test):
compile writes <kernel>.hsaco (ELF, symbol = kernel name) and .isa, prints
`wrote ...` lines and `compile ok`; a bogus --target exits 1 listing the valid
targets; no arguments exits 2; bench without a GPU skips with 77. Each
compiled artifact carries the instructions its kernel's design depends on
(MFMA, direct-to-LDS loads, DPP reductions, exp/rsq) and no spills. On the
GPU: one timed row and the G32 results.csv schema, comparator rows, tune,
and the reference's e2e flow (compile through the CLI, load the written
.hsaco, launch with the reference geometry, compare with the fp64 oracle)."""
import csv
import os
import subprocess

import pytest

import kernelh as kh

CLI = kh.CLI_PATH


def run(*args, cwd=None):
    return subprocess.run([CLI, *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, cwd=cwd,
                          timeout=120)


@pytest.mark.parametrize("kernel,shape", [("vecadd", "n=1024"), ("softmax", "rows=4096,cols=1024"),
                                          ("scan_totals", "n=1000000"),
                                          ("attention", "batch=4,heads=16,seq=4096,head_dim=64")])
def test_compile_writes_artifacts(tmp_path, kernel, shape):
    r = run("compile", "--kernel", kernel, "--shape", shape, "--target", "amdgcn-gfx950", "--out", str(tmp_path),
            "--resources")
    assert r.returncode == 0, r.stdout
    lines = r.stdout.splitlines()
    assert lines[0] == f"wrote {tmp_path}/{kernel}.hsaco"
    assert lines[-1] == "compile ok"
    blob = (tmp_path / f"{kernel}.hsaco").read_bytes()
    assert blob[:4] == b"\x7fELF" and (kernel + ".kd").encode() in blob
    isa = (tmp_path / f"{kernel}.isa").read_text()
    assert "s_waitcnt" in isa and kernel in isa
    res = (tmp_path / "resources.json").read_text()
    assert '"wavefront_size": 64' in res and '"target": "amdgcn-gfx950"' in res


# What each kernel's design depends on, probed in the compiled artifact the
# way the reference's degraded-mode e2e tests probe theirs for ds_ / exp_f32
# / rsq (e2e_gemm_test.cpp:211-231, e2e_layernorm_test.cpp:274-292).
DESIGN_INSTRUCTIONS = {
    # Streaming kernels: nontemporal dwordx4 buffer accesses over row / step spans.
    "vecadd": ("n=16777216", ["buffer_load_dwordx4", "buffer_store_dwordx4", "offen nt"]),
    "fused_gelu": ("n=67108864", ["v_exp_f32", "v_rcp_f32", "buffer_load_dwordx4", "offen nt"]),
    "softmax": ("rows=4096,cols=1024", ["v_exp_f32", "row_ror:8", "buffer_load_dwordx4", "offen nt"]),
    "layernorm": ("rows=4096,cols=1024", ["v_rsq_f32", "row_ror:8", "buffer_load_dwordx4", "offen nt"]),
    "scan": ("n=67108864", ["row_shr:8", "row_bcast:31", "global_atomic_add", "buffer_load_dwordx4"]),
    "gemm": ("m=8192,n=8192,k=8192", ["v_mfma_f32_32x32x2_f32", "offen lds", "ds_read_b128", "s_setprio"]),
    "attention": ("batch=4,heads=16,seq=4096,head_dim=64", ["v_mfma_f32_32x32x2_f32", "v_exp_f32", "ds_read_b128"]),
}


@pytest.mark.parametrize("kernel", sorted(DESIGN_INSTRUCTIONS))
def test_compiled_isa_carries_the_design_instructions(tmp_path, kernel):
    shape, needles = DESIGN_INSTRUCTIONS[kernel]
    r = run("compile", "--kernel", kernel, "--shape", shape, "--out", str(tmp_path), "--resources")
    assert r.returncode == 0, r.stdout
    isa = (tmp_path / f"{kernel}.isa").read_text()
    missing = [n for n in needles if n not in isa]
    assert not missing, f"{kernel}.isa lacks {missing}"
    res = (tmp_path / "resources.json").read_text()
    assert '"scratch_bytes": 0' in res  # no register spills


@pytest.mark.parametrize("kernel", sorted(DESIGN_INSTRUCTIONS) + ["scan_totals"])
def test_resources_json_reference_schema(tmp_path, kernel):
    """resources.json parses as JSON and carries the reference's contract keys
    with their types (resource_reporter.hpp:50-58); occupancy_estimate is the
    reference's register-limited waves per CU (resource_reporter.cpp:232-255)
    over gfx950's register file of 4 SIMDs x 512 registers x 64 lanes, capped
    at 32 waves. The hardware allocates registers in granules of 8, 4 SIMDs
    of 512 each, so its resident count, 4 * floor(512 / roundup8(registers)),
    is never above the estimate and equals it on a multiple of 8 below 64."""
    import json
    shape = DESIGN_INSTRUCTIONS.get(kernel, ("n=1000000",))[0]
    r = run("compile", "--kernel", kernel, "--shape", shape, "--out", str(tmp_path), "--resources")
    assert r.returncode == 0, r.stdout
    res = json.loads((tmp_path / "resources.json").read_text())
    for key, typ in (("kernel", str), ("target", str), ("vgpr_count", int), ("sgpr_count", int),
                     ("lds_bytes", int), ("wavefront_size", int), ("occupancy_estimate", int)):
        assert isinstance(res[key], typ), (key, res.get(key))
    assert res["kernel"] == kernel and res["target"] == "amdgcn-gfx950" and res["wavefront_size"] == 64
    regs = res["vgpr_count"] + res["agpr_count"]
    assert 0 < regs <= 512
    est = res["occupancy_estimate"]
    assert est == min(32, max(1, (4 * 512 * 64) // (regs * 64)))
    hw = min(32, 4 * (512 // (-(-regs // 8) * 8)))
    assert hw <= est and (regs % 8 or regs >= 64 or hw == est)
    # The launch the launcher makes at this shape fits those waves.
    threads = res["launch"]["block"][0] * res["launch"]["block"][1] * res["launch"]["block"][2]
    assert res["occupancy_estimate"] * 64 >= threads


def test_compile_bogus_target_exit_1(tmp_path):
    r = run("compile", "--kernel", "vecadd", "--shape", "n=1024", "--target", "bogus-target", "--out", str(tmp_path))
    assert r.returncode == 1
    assert "error: unknown device target" in r.stdout
    assert "error: valid --target values: amdgcn-gfx950" in r.stdout


def test_compile_reference_target_refused(tmp_path):
    r = run("compile", "--kernel", "vecadd", "--shape", "n=1024", "--target", "amdgcn-gfx1101", "--out", str(tmp_path))
    assert r.returncode == 1 and "gfx950 code objects only" in r.stdout


def test_usage_errors_exit_2(tmp_path):
    assert run("compile").returncode == 2
    assert run().returncode == 2
    assert run("compile", "--kernel", "vecadd", "--out", str(tmp_path)).returncode == 2  # no --shape
    assert run("compile", "--kernel", "vecadd", "--shape", "n", "--out", str(tmp_path)).returncode == 2
    assert run("bench").returncode == 2  # no --out
    assert run("bench", "--suite", "cuda-cross", "--out", str(tmp_path)).returncode == 2  # not built here
    assert run("bench", "--kernel", "gemm", "--shape", "m=8,n=8,k=8", "--backend", "cublas",
               "--out", str(tmp_path)).returncode == 2
    assert run("--help").returncode == 0


def test_compile_bad_shape_and_unknown_kernel_exit_1(tmp_path):
    r = run("compile", "--kernel", "softmax", "--shape", "rows=4", "--out", str(tmp_path))
    assert r.returncode == 1 and "'rows' and 'cols' are required" in r.stdout
    r = run("compile", "--kernel", "matmul", "--shape", "n=4", "--out", str(tmp_path))
    assert r.returncode == 1 and "registered kernels:" in r.stdout


def test_bench_without_gpu_skips_77(tmp_path):
    if kh.device_count() > 0:
        pytest.skip("a device is visible")
    r = run("bench", "--suite", "kernelh", "--out", str(tmp_path), "--occupancy")
    assert r.returncode == 77
    assert (tmp_path / "occupancy.md").exists() and (tmp_path / "occupancy.json").exists()


@pytest.mark.gpu
def test_bench_single_row_results_csv(dev, tmp_path):
    print("[gpu-case] kernelh bench --kernel vecadd", flush=True)
    r = run("bench", "--kernel", "vecadd", "--shape", "n=1048576", "--out", str(tmp_path), "--occupancy")
    assert r.returncode == 0, r.stdout
    rows = list(csv.DictReader(open(tmp_path / "results.csv")))
    assert list(rows[0].keys()) == ["kernel", "shape", "backend", "ms_median", "gflops_or_gbps", "timestamp", "device"]
    assert rows[0]["kernel"] == "vecadd" and rows[0]["backend"] == "kernelh"
    assert float(rows[0]["ms_median"]) > 0 and float(rows[0]["gflops_or_gbps"]) > 100
    assert "gfx950" in rows[0]["device"]
    occ = (tmp_path / "occupancy.md").read_text()
    assert "| vecadd |" in occ


@pytest.mark.gpu
@pytest.mark.parametrize("kernel,shape,backend", [
    ("gemm", "m=512,n=512,k=512", "rocblas"),
    ("gemm", "m=512,n=512,k=512", "hipblaslt"),
    ("gemm", "m=512,n=512,k=512", "hipref-naive"),
    ("softmax", "rows=4096,cols=1024", "hipref-vec"),
    ("scan", "n=100000", "hipref-naive"),
    ("roofline_fma", "n=4194304", "roofline"),
])
def test_bench_comparator_rows(dev, tmp_path, kernel, shape, backend):
    # The reference's comparator backends (bench/harness/run_bench.cpp:48-66)
    # produce rows in the same results.csv.
    print(f"[gpu-case] kernelh bench --kernel {kernel} --backend {backend}", flush=True)
    r = run("bench", "--kernel", kernel, "--shape", shape, "--backend", backend, "--out", str(tmp_path))
    assert r.returncode == 0, r.stdout
    rows = list(csv.DictReader(open(tmp_path / "results.csv")))
    assert rows[0]["backend"] == backend and float(rows[0]["gflops_or_gbps"]) > 0


def test_tune_usage_and_refusals(tmp_path):
    # kernelh tune (tools/kernelh/main.cpp:649-760, 1320-1350): usage errors
    # exit 2, unsupported kernel / target exit 1, no device exits 77.
    assert run("tune", "--out", str(tmp_path)).returncode == 2                       # no --shape
    assert run("tune", "--shape", "m=8,n=8,k=8").returncode == 2                     # no --out
    assert run("tune", "--shape", "m=8,n=8,k=8", "--out", str(tmp_path), "--max-candidates", "0").returncode == 2
    assert run("tune", "--shape", "m=8,n=8,k=8", "--out", str(tmp_path), "--timeout", "9999").returncode == 2
    r = run("tune", "--kernel", "softmax", "--shape", "m=8,n=8,k=8", "--out", str(tmp_path))
    assert r.returncode == 1 and "only the 'gemm' kernel" in r.stdout
    r = run("tune", "--shape", "m=8,n=8,k=8", "--out", str(tmp_path), "--target", "amdgcn-gfx1101")
    assert r.returncode == 1 and "amdgcn-gfx950" in r.stdout
    if kh.device_count() == 0:
        assert run("tune", "--shape", "m=8,n=8,k=8", "--out", str(tmp_path)).returncode == 77


@pytest.mark.gpu
def test_tune_evaluates_candidates_and_caches(dev, tmp_path):
    print("[gpu-case] kernelh tune gemm m=n=k=512, 10 candidates", flush=True)
    cache = str(tmp_path / "cache.json")
    shape = "m=512,n=512,k=512"
    args = ("tune", "--shape", shape, "--out", str(tmp_path), "--max-candidates", "10",
            "--timeout", "60", "--cache", cache)
    r = run(*args)
    assert r.returncode == 0, r.stdout
    assert "best config: gemm" in r.stdout and "tune ok" in r.stdout
    rows = list(csv.DictReader(open(tmp_path / "tune-results.csv")))
    assert len(rows) == 10
    assert list(rows[0].keys())[:11] == ["kernel", "shape", "bm", "bn", "bk", "waves", "unroll", "vec", "ms_median",
                                          "accepted", "reason"]
    assert all(row["accepted"] == "true" and row["reason"] == "ok" for row in rows), rows
    assert all(float(row["ms_median"]) > 0 for row in rows)
    # The launcher's own symbols come first, with their real axes: the
    # persistent 128x256 `gemm` (4 waves, two slabs ahead), the K-split
    # symbols (8 waves; the deep one three batches ahead).
    by = {row["symbol"]: row for row in rows}
    assert (by["gemm"]["bm"], by["gemm"]["bn"], by["gemm"]["waves"], by["gemm"]["unroll"]) == ("128", "256", "4", "2")
    assert (by["gemm_mid"]["unroll"], by["gemm_ksplit"]["waves"], by["gemm_ksplit_deep"]["unroll"]) == ("1", "8", "3")
    assert {row["vec"] for row in rows} == {"4"}  # k, n multiples of 4: dwordx4 loads
    assert all(row["product"] == ("1" if i < 7 else "0") for i, row in enumerate(rows))
    best = min(rows, key=lambda row: float(row["ms_median"]))["symbol"]
    assert f"best config: {best} " in r.stdout
    r2 = run(*args)
    assert r2.returncode == 0 and "cache-hit" in r2.stdout and "served from cache" in r2.stdout
    # The runtime's launcher reads the same cache: kh_gemm then runs `best`.
    kh.set_tune_cache(cache)
    try:
        assert kh.launch_symbol("gemm", shape) == best
    finally:
        kh.set_tune_cache(None)


@pytest.mark.gpu
def test_tune_sampled_search(dev, tmp_path):
    """--sample n evaluates n candidates in a fixed pseudo-random order, then
    --refine-budget r at most r more, each one design step from the best
    accepted one of the sample; the same flags give the same candidates."""
    print("[gpu-case] kernelh tune gemm m=n=k=256 --sample 6 --refine-budget 3", flush=True)
    shape = "m=256,n=256,k=256"
    symbols = []
    for rep in range(2):
        out = tmp_path / f"r{rep}"
        r = run("tune", "--shape", shape, "--out", str(out), "--sample", "6", "--refine-budget", "3",
                "--timeout", "60", "--cache", str(tmp_path / f"cache{rep}.json"))
        assert r.returncode == 0, r.stdout
        rows = list(csv.DictReader(open(out / "tune-results.csv")))
        assert 6 <= len(rows) <= 9 and len({row["symbol"] for row in rows}) == len(rows)
        symbols.append([row["symbol"] for row in rows])
        sample = rows[:6]
        centre = min((row for row in sample if row["accepted"] == "true"), key=lambda row: float(row["ms_median"]))
        assert f"refining around {centre['symbol']} with {len(rows) - 6} neighbour(s)" in r.stdout
        axes = ("bm", "bn", "bk", "waves", "unroll", "mfma", "pipeline", "prio")
        cand = {c["symbol"]: c for c in kh.gemm_candidates()}
        for row in rows[6:]:
            a, b = cand[row["symbol"]], cand[centre["symbol"]]
            diffs = sum(a[x] != b[x] for x in axes) + (a["k_split"] != b["k_split"])
            assert diffs == 1, (row["symbol"], centre["symbol"])
    assert symbols[0] == symbols[1]


@pytest.mark.gpu
def test_tune_vec_column_follows_the_shape(dev, tmp_path):
    # k not a multiple of 4: every candidate takes its guarded scalar loads.
    print("[gpu-case] kernelh tune gemm m=100,n=100,k=33, 2 candidates", flush=True)
    r = run("tune", "--shape", "m=100,n=100,k=33", "--out", str(tmp_path), "--max-candidates", "2",
            "--cache", str(tmp_path / "c.json"))
    assert r.returncode == 0, r.stdout
    rows = list(csv.DictReader(open(tmp_path / "tune-results.csv")))
    assert [row["vec"] for row in rows] == ["1", "1"]
    assert all(row["accepted"] == "true" for row in rows), rows


@pytest.mark.gpu
@pytest.mark.parametrize("kernel", ["vecadd", "softmax", "gemm", "scan"])
def test_cli_compiled_code_object_runs_under_reference_geometry(dev, tmp_path, kernel):
    """The reference's e2e flow (e2e_*_test.cpp): compile through the CLI,
    load the written <kernel>.hsaco with hipModuleLoadData, launch it with
    the reference's own geometry and check it against the fp64 reference."""
    import numpy as np
    import oracle as O
    from khtest import down, empty, up
    shapes = {"vecadd": "n=100000", "softmax": "rows=257,cols=1000", "gemm": "m=300,n=200,k=100", "scan": "n=100000"}
    r = run("compile", "--kernel", kernel, "--shape", shapes[kernel], "--out", str(tmp_path))
    assert r.returncode == 0, r.stdout
    mod = kh.GpuModule((tmp_path / f"{kernel}.hsaco").read_bytes())
    f = mod.get_function(kernel)
    print(f"[gpu-case] {kernel} from kernelh compile, reference geometry", flush=True)
    if kernel == "vecadd":
        n = 100000
        a, b = O.vecadd_inputs(n)
        da, db, dc = up(a), up(b), empty(n)
        args = kh.LaunchArgs().add_memref(da, [n]).add_memref(db, [n]).add_memref(dc, [n])
        kh.kernel_launch(f, ((n + 255) // 256, 1, 1), (256, 1, 1), args)
        assert np.array_equal(down(dc, n), O.ref_vecadd(a, b))
    elif kernel == "softmax":
        rows, cols = 257, 1000
        x, _ = O.lcg_fill(rows * cols, 0x27AB13)
        dx, dy = up(x), empty(rows * cols)
        args = kh.LaunchArgs().add_memref(dx, [rows, cols]).add_memref(dy, [rows, cols])
        kh.kernel_launch(f, (rows, 1, 1), (256, 1, 1), args)
        assert np.max(np.abs(down(dy, rows * cols) - O.ref_softmax(x, rows, cols).ravel())) <= 1e-4
    elif kernel == "gemm":
        m, n, k = 300, 200, 100
        A, B = O.gemm_int_inputs(m, n, k)
        dA, dB, dC = up(A), up(B), empty(m * n)
        args = kh.LaunchArgs().add_memref(dA, [m, k]).add_memref(dB, [k, n]).add_memref(dC, [m, n])
        kh.kernel_launch(f, ((m + 31) // 32, 1, 1), (256, 1, 1), args)
        ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)  # exact integers
        assert np.array_equal(down(dC, m * n).reshape(m, n), ref)
    else:
        n = 100000
        T = (n + 255) // 256
        x = O.mt19937_fill(n, 0x29C0FFEE)
        dx, dy, dyl = up(x), empty(n), empty(n)
        dth, dtl = empty(T, None), empty(T, None)  # totals as hipMalloc left them
        args = kh.LaunchArgs()
        for buf, c in ((dx, n), (dy, n), (dyl, n), (dth, T), (dtl, T)):
            args.add_memref(buf, [c])
        # The template's pass-1 geometry, launched alone and unverified, as
        # the reference's HipBackend::launch_kernel does.
        kh.launch_raw(f, (T, 1, 1), (256, 1, 1), args)
        assert np.array_equal(down(dy, n), O.ref_scan(x).astype(np.float32))


# ------------------------------------------------------------------ occupancy-only mode

@pytest.mark.parametrize("kernel,shape", [("gemm", None), ("softmax", None), ("scan", None), ("attention", None),
                                          ("vecadd", None), ("fused_gelu", None), ("layernorm", None),
                                          ("gemm", "m=8192,n=8192,k=8192")])
def test_bench_occupancy_only_mode(tmp_path, kernel, shape):
    """`bench --occupancy --kernel <k> --target <t> [--shape] --out d` times
    nothing and needs no device: exit 0 and occupancy.{json,md} for that one
    kernel (run_bench.cpp:111-127), with the reference's report keys
    (occupancy.cpp:90-110) at the reference's default shapes
    (kernelh_backend.cpp:447-469) unless --shape names one."""
    import json
    args = ["bench", "--occupancy", "--kernel", kernel, "--target", "amdgcn-gfx950", "--out", str(tmp_path)]
    if shape:
        args += ["--shape", shape]
    r = run(*args)
    assert r.returncode == 0, r.stdout
    assert f"wrote {tmp_path}/occupancy.json + occupancy.md ({kernel}, amdgcn-gfx950)" in r.stdout
    rep = json.loads((tmp_path / "occupancy.json").read_text())
    for key in ("kernel", "target", "config", "vgpr_count", "lds_bytes", "threads_per_workgroup",
                "vgpr_limited_waves", "lds_limited_blocks", "thread_limited_blocks", "theoretical_waves",
                "theoretical_pct", "limiter", "measured_blocks", "measured_pct", "measured_note"):
        assert key in rep, key
    defaults = {"gemm": "m=512,n=512,k=512", "softmax": "rows=4096,cols=1024", "scan": "n=100000",
                "attention": "batch=2,heads=8,seq=512,head_dim=64", "vecadd": "n=1024",
                "fused_gelu": "n=1048576", "layernorm": "rows=4096,cols=1024"}
    assert rep["kernel"] == kernel and rep["target"] == "amdgcn-gfx950"
    assert rep["config"] == (shape or defaults[kernel])
    # The symbol the launcher runs at that shape, with its own resources and
    # workgroup size, through the pinned formulas.
    sym = kh.launch_symbol(kernel, rep["config"])
    res = kh.resources(sym)
    grid, block = kh.geometry(kernel, rep["config"])
    assert rep["symbol"] == sym
    assert rep["vgpr_count"] == res["vgpr_count"] + res["agpr_count"] and rep["lds_bytes"] == res["lds_bytes"]
    assert rep["threads_per_workgroup"] == block[0] * block[1] * block[2]
    ref = kh.occupancy(rep["vgpr_count"], rep["lds_bytes"], rep["threads_per_workgroup"])
    assert rep["theoretical_waves"] == ref.achieved_waves
    if kh.device_count() == 0:
        assert rep["measured_blocks"] == -1 and "analytic only" in rep["measured_note"]
    md = (tmp_path / "occupancy.md").read_text()
    assert f"| {kernel} | {rep['config']} | {sym} |" in md


def test_bench_occupancy_only_threads_override(tmp_path):
    r = run("bench", "--occupancy", "--kernel", "attention", "--target", "amdgcn-gfx950", "--threads", "64",
            "--out", str(tmp_path))
    assert r.returncode == 0, r.stdout
    import json
    rep = json.loads((tmp_path / "occupancy.json").read_text())
    assert rep["threads_per_workgroup"] == 64
    assert rep["thread_limited_blocks"] == 1024 // 64


@pytest.mark.parametrize("args,code,msg", [
    (["--occupancy", "--kernel", "gemm", "--target", "amdgcn-gfx1101"], 2, "unknown --target 'amdgcn-gfx1101'"),
    (["--occupancy", "--kernel", "gemm", "--target", "amdgcn-gfx950", "--threads", "0"], 2,
     "--threads must be an integer in [1,1048576]"),
    (["--occupancy", "--kernel", "gemm", "--target", "amdgcn-gfx950", "--threads", "1048577"], 2,
     "--threads must be an integer in [1,1048576]"),
    (["--occupancy", "--kernel", "gemm", "--target", "amdgcn-gfx950", "--shape", "m=8,n"], 2, "malformed --shape"),
    (["--target", "amdgcn-gfx950"], 2, "--target/--threads require --occupancy"),
    (["--threads", "64"], 2, "--target/--threads require --occupancy"),
    (["--occupancy", "--kernel", "gemm"], 2, "--target amdgcn-gfx950"),
    (["--occupancy", "--kernel", "conv2d", "--target", "amdgcn-gfx950"], 1, "no default shape"),
    (["--occupancy", "--kernel", "gemm", "--target", "amdgcn-gfx950", "--shape", "m=8"], 1, "required"),
])
def test_bench_occupancy_only_errors(tmp_path, args, code, msg):
    r = run("bench", *args, "--out", str(tmp_path))
    assert r.returncode == code, r.stdout
    assert msg in r.stdout


# ------------------------------------------------------------------ tune search flags

@pytest.mark.parametrize("flag,value", [("--sample", "0"), ("--sample", "217"), ("--sample", "x"),
                                        ("--refine-budget", "-1"), ("--refine-budget", "81"),
                                        ("--max-candidates", "0"), ("--timeout", "3601")])
def test_tune_flag_ranges_exit_2(tmp_path, flag, value):
    r = run("tune", "--shape", "m=64,n=64,k=64", "--out", str(tmp_path), flag, value)
    assert r.returncode == 2
    assert f"error: {flag} must be an integer in [" in r.stdout


def test_tune_search_flags_accepted(tmp_path):
    """The reference's documented search flags (main.cpp:704-730) in range:
    never a usage error; without a device the run skips with 77."""
    for extra in (["--sample", "1"], ["--sample", "216"], ["--refine-budget", "0"], ["--refine-budget", "80"],
                  ["--sample", "20", "--refine-budget", "4", "--max-candidates", "24"]):
        r = run("tune", "--kernel", "gemm", "--shape", "m=64,n=64,k=64", "--out", str(tmp_path), *extra)
        assert r.returncode in (0, 77), (extra, r.stdout)
        if kh.device_count() == 0:
            assert r.returncode == 77 and "skip: no HIP device" in r.stdout
