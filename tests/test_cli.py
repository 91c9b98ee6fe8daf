"""The `kernelh` CLI contract (tools/kernelh/main.cpp; test/lit/cli/compile.test):
compile writes <kernel>.hsaco (ELF, symbol = kernel name) and .isa, prints
`wrote ...` lines and `compile ok`; a bogus --target exits 1 listing the valid
targets; no arguments exits 2; bench without a GPU skips with 77. The GPU
test runs one timed row and checks the G32 results.csv schema."""
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
    print("[gpu-case] kernelh tune gemm m=n=k=512, 6 candidates", flush=True)
    cache = str(tmp_path / "cache.json")
    args = ("tune", "--shape", "m=512,n=512,k=512", "--out", str(tmp_path), "--max-candidates", "6",
            "--timeout", "60", "--cache", cache)
    r = run(*args)
    assert r.returncode == 0, r.stdout
    assert "best config: gemm_t" in r.stdout and "tune ok" in r.stdout
    rows = list(csv.DictReader(open(tmp_path / "tune-results.csv")))
    assert len(rows) == 6
    assert list(rows[0].keys())[:11] == ["kernel", "shape", "bm", "bn", "bk", "waves", "unroll", "vec", "ms_median",
                                          "accepted", "reason"]
    assert all(row["accepted"] == "true" and row["reason"] == "ok" for row in rows), rows
    assert all(float(row["ms_median"]) > 0 for row in rows)
    r2 = run(*args)
    assert r2.returncode == 0 and "cache-hit" in r2.stdout and "served from cache" in r2.stdout
