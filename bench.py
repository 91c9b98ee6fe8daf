#!/usr/bin/env python3
"""Benchmark of the kernel.h seven-template hot path on one MI355X.

One step = one pass of the suite the BASELINE metric is quoted on, at the
BASELINE sizes: gemm 8192^3 (the headline `value`, fp32 TFLOP/s), softmax
4096x1024 and scan 2^26 (HBM GB/s), plus vecadd 2^24, layernorm 4096x1024,
fused_gelu 2^26 and attention b4 h16 s4096 d64, each reported under
"kernels". Inputs are synthetic (numpy generators), resident in HBM before
the timed region; every launch goes through the khrt C-ABI
(hipModuleLaunchKernel on the embedded gfx950 code objects).

Timing: W untimed warmup steps, then K timed steps bracketed by device
synchronisation. Per kernel, HIP events recorded on the launch stream around
its K back-to-back launches give the average launch duration. Working sets
smaller than 1 GiB rotate over several buffer sets so every launch reads
from HBM rather than the 256 MB Infinity Cache.

Roofline: `achieved` = algorithmic bytes (or FLOPs) per launch / average
launch duration; `peak` = MI355X published peak (HBM 8 TB/s; fp32 MFMA
157.3 TFLOP/s). The CPU baseline times the oracle's fp64 reference on a
bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "kernel.h_amd"))

import numpy as np  # noqa: E402

HBM_PEAK_GBPS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
ROTATE_BYTES = 1 << 30  # rotate buffer sets until the working set exceeds 1 GiB

METRIC = "GEMM-8192 fp32 TFLOPS + softmax/scan HBM GB/s, % of MI355X roofline"

# HBM bytes per launch from two rocprofv3 --pmc passes (FETCH_SIZE scaled by
# 2.000 and WRITE_SIZE by 1.000, the factors a copy kernel of known size
# reads), recorded in profiles/templates_baseline_sizes_hbm_traffic.md.
PMC_TRAFFIC_BYTES = {
    "vecadd": 201374080, "softmax": 33634176, "layernorm": 33737882, "scan": 539377210,
    "fused_gelu": 537017626, "gemm": 4281652941, "attention": 1208230925,
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def u24(rng, n, lo, hi):
    """Uniform on the 2^-24 grid, lo + (hi-lo) u, rounded to fp32."""
    u = rng.integers(0, 1 << 24, n, dtype=np.int64).astype(np.float64) / float(1 << 24)
    return (lo + (hi - lo) * u).astype(np.float32)


def normal(rng, n, sd):
    return (rng.standard_normal(n) * sd).astype(np.float32)


class Case:
    """One template at one BASELINE configuration."""

    def __init__(self, name, config, work, unit, bound, setup, launch, traffic_note=""):
        self.name, self.config, self.work, self.unit, self.bound = name, config, work, unit, bound
        self.setup, self.launch, self.traffic_note = setup, launch, traffic_note
        self.sets = []
        self.ms = []


def make_cases(kh, rng, only):
    up = lambda a: kh.Buffer.from_array(a)
    cases = []

    def add(c):
        if only is None or c.name in only:
            cases.append(c)

    n = 1 << 24
    add(Case("vecadd", "n=2^24 fp32, a,b ~ U[-1,1]", 12.0 * n, "GB/s", "hbm",
             lambda: (up(u24(rng, n, -1, 1)), up(u24(rng, n, -1, 1)), kh.Buffer(4 * n)),
             lambda s, st: kh.vecadd(s[0], s[1], s[2], n, st)))

    R, C = 4096, 1024
    add(Case("softmax", "4096x1024 fp32, x ~ N(0, 4^2)", 8.0 * R * C, "GB/s", "hbm",
             lambda: (up(normal(rng, R * C, 4.0)), kh.Buffer(4 * R * C)),
             lambda s, st: kh.softmax(s[0], s[1], R, C, st)))

    add(Case("layernorm", "4096x1024 fp32, eps 1e-5, x ~ N(0, 4^2), gamma U[0.5,1.5], beta U[-0.1,0.1]",
             8.0 * R * C + 8.0 * C, "GB/s", "hbm",
             lambda: (up(normal(rng, R * C, 4.0)), up(u24(rng, C, 0.5, 1.5)), up(u24(rng, C, -0.1, 0.1)),
                      kh.Buffer(4 * R * C)),
             lambda s, st: kh.layernorm(s[0], s[1], s[2], s[3], R, C, st)))

    ns = 1 << 26
    T = kh.scan_workspace_floats(ns)
    add(Case("scan", "inclusive n=2^26 fp32, x ~ U[0,1) on the 2^-24 grid", 8.0 * ns, "GB/s", "hbm",
             lambda: (up(u24(rng, ns, 0, 1)), kh.Buffer(4 * ns), kh.Buffer(4 * T), kh.Buffer(4 * T)),
             lambda s, st: kh.scan(s[0], s[1], None, s[2], s[3], ns, st)))

    ng = 1 << 26
    add(Case("fused_gelu", "n=2^26 fp32, x ~ N(0,1); out = gelu_tanh(1.5x+0.5)", 8.0 * ng, "GB/s", "hbm",
             lambda: (up(normal(rng, ng, 1.0)), kh.Buffer(4 * ng)),
             lambda s, st: kh.fused_gelu(s[0], None, s[1], ng, st),
             "reference formula counts 12 B/elem (metrics.cpp:36-38); 8 B/elem are moved"))

    M = 8192
    add(Case("gemm", "C=A*B fp32 row-major, m=n=k=8192, A,B ~ U[-1,1]", 2.0 * M * M * M, "TFLOP/s", "mfma",
             lambda: (up(u24(rng, M * M, -1, 1)), up(u24(rng, M * M, -1, 1)), kh.Buffer(4 * M * M)),
             lambda s, st: kh.gemm(s[0], s[1], s[2], M, M, M, st)))

    b, h, s_, d = 4, 16, 4096, 64
    add(Case("attention", "non-causal b=4 h=16 s=4096 d=64 fp32, Q,K,V ~ N(0,1)", 4.0 * b * h * s_ * s_ * d,
             "TFLOP/s", "mfma",
             lambda: tuple(up(normal(rng, b * h * s_ * d, 1.0)) for _ in range(3)) + (kh.Buffer(4 * b * h * s_ * d),),
             lambda s, st: kh.attention(s[0], s[1], s[2], s[3], b, h, s_, d, st)))
    return cases


def measure_ceilings(kh, stream, reps=5):
    """Measured roofline denominators: triad and copy over 2^28 floats per
    buffer (3 GiB / 2 GiB moved per launch, beyond the 256 MB MALL, as the
    reference's roofline_triad, bench/harness/roofline.cpp:60-84) and the
    fp32 MFMA microbenchmark (8 independent chains per wave, two waves per
    SIMD, ~2 ms per launch: shorter launches under-measure it, as the clock
    has not settled and launch gaps count)."""
    n = 1 << 28
    a, b, c = kh.Buffer(4 * n), kh.Buffer(4 * n), kh.Buffer(4 * n)
    a.fill(1.0, stream)
    b.fill(2.0, stream)
    e0, e1 = kh.Event(), kh.Event()

    def timed(fn):
        fn()
        stream.synchronize()
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_ms(e1) / reps

    t_triad = timed(lambda: kh.roofline_triad(a, b, c, n, stream))
    t_copy = timed(lambda: kh.roofline_copy(a, c, n, stream))
    cu = kh.device_info()["cu_count"]
    blocks, iters = cu * 2, 4096
    out = kh.Buffer(4 * blocks * 256)
    flops = float(blocks) * 4 * iters * 8 * 4096
    t_mfma = timed(lambda: kh.roofline_mfma(out, blocks, iters, stream))
    for buf in (a, b, c, out):
        buf.free()
    return {"hbm_triad_gbps": 12.0 * n / (t_triad * 1e-3) / 1e9,
            "hbm_copy_gbps": 8.0 * n / (t_copy * 1e-3) / 1e9,
            "fp32_mfma_tflops": flops / (t_mfma * 1e-3) / 1e12,
            "triad_bytes_per_launch": 12 * n, "copy_bytes_per_launch": 8 * n,
            "mfma_config": f"{blocks} workgroups x 4 waves x {iters} x 8 v_mfma_f32_32x32x2f32"}


def available(kh, name):
    try:
        kh.code_object(name)
        return True
    except kh.KhrtError:
        return False


def set_bytes(sets):
    return sum(b.nbytes for b in sets)


def _gemm_rows_rate(O, A, B, M, threads, budget_s):
    """Grows a row sample of the 8192^3 fp64 GEMM reference until it has run
    for about budget_s seconds; returns (TFLOP/s, rows, seconds)."""
    O.set_threads(threads)
    done, dt, rows = 0, 0.0, max(threads, 2)
    while dt < budget_s and done < M:
        rows = min(rows, M - done)
        t = time.perf_counter()
        O.ref_gemm(A, B, M, M, M, row0=done, nrows=rows)
        dt += time.perf_counter() - t
        done += rows
        rows = max(rows, int(rows * min(4.0, 0.9 * (budget_s - dt) / max(time.perf_counter() - t, 1e-3))))
    return 2.0 * done * M * M / dt / 1e12, done, dt


def cpu_baseline(budget_s: float):
    """The oracle's fp64 references (CPU restatements of the reference's
    e2e checks) timed on this host: the GEMM reference (e2e_gemm_test.cpp:
    92-110) on a row sample of the 8192^3 problem on all cores via OpenMP
    (the headline, in `value`'s unit) and on one core, plus all-core rates
    of the softmax and scan references at the BASELINE sizes."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    cores = len(os.sched_getaffinity(0))
    M = 8192
    rng = np.random.default_rng(7)
    A = u24(rng, M * M, -1, 1)
    B = u24(rng, M * M, -1, 1)
    tf_all, rows_all, s_all = _gemm_rows_rate(O, A, B, M, cores, 0.6 * budget_s)
    tf_one, rows_one, s_one = _gemm_rows_rate(O, A, B, M, 1, 0.25 * budget_s)
    del A, B
    O.set_threads(cores)
    x = (rng.standard_normal(4096 * 1024) * 4.0).astype(np.float32)
    t = time.perf_counter()
    O.ref_softmax(x, 4096, 1024)
    sm = 8.0 * x.size / (time.perf_counter() - t) / 1e9
    xs = u24(rng, 1 << 26, 0, 1)
    t = time.perf_counter()
    O.ref_scan(xs)
    sc = 8.0 * xs.size / (time.perf_counter() - t) / 1e9
    return {"value": tf_all, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"fp64 rank-1 GEMM reference (oracle kho_ref_gemm): {rows_all} of 8192 rows of the "
                      f"8192^3 problem in {s_all:.1f} s on {cores} threads",
            "single_thread": {"value": tf_one, "unit": "TFLOP/s", "cores": 1,
                              "sample": f"{rows_one} rows in {s_one:.1f} s"},
            "other_kernels": {"softmax_4096x1024_gbps": sm, "scan_2^26_gbps_single_thread": sc,
                              "note": "fp64 references, same inputs as the GPU rows; scan is serial"}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--kernels", default="", help="comma list to restrict the suite")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--no-rotate", action="store_true", help="reuse one buffer set (cache-warm)")
    ap.add_argument("--no-ceilings", action="store_true", help="skip the measured roofline microbenchmarks")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}); "
              "multi-GPU runs are out of scope", file=sys.stderr)
        return 2

    import kernelh as kh
    kh.init_device(0)
    info = kh.device_info()
    log(f"[bench] device {info['name']} {info['arch']} cu={info['cu_count']}")
    rng = np.random.default_rng(20261201)
    only = set(a.kernels.split(",")) if a.kernels else None
    cases = [c for c in make_cases(kh, rng, only) if available(kh, c.name)]
    stream = kh.Stream()

    for c in cases:
        c.sets = [c.setup()]
        if not a.no_rotate:
            while set_bytes([b for s in c.sets for b in s]) < ROTATE_BYTES and len(c.sets) < 64:
                c.sets.append(c.setup())
        log(f"[bench] {c.name}: {len(c.sets)} buffer set(s), "
            f"{set_bytes([b for s in c.sets for b in s]) / 2**20:.0f} MiB")

    ev = {c.name: (kh.Event(), kh.Event()) for c in cases}
    kh.synchronize()

    for i in range(a.warmup):
        for c in cases:
            c.launch(c.sets[i % len(c.sets)], stream)
    stream.synchronize()
    log(f"[bench] warmup done ({a.warmup} steps)")

    # Timed region: the K steps are issued kernel-major, so each kernel's K
    # launches run back to back between one pair of events on the launch
    # stream (average launch duration = elapsed / K, no host gaps).
    kh.synchronize()
    t0 = time.perf_counter()
    for c in cases:
        e0, e1 = ev[c.name]
        e0.record(stream)
        for i in range(a.steps):
            c.launch(c.sets[(a.warmup + i) % len(c.sets)], stream)
        e1.record(stream)
    stream.synchronize()
    kh.synchronize()
    wall = time.perf_counter() - t0
    for c in cases:
        e0, e1 = ev[c.name]
        c.ms_host = e0.elapsed_ms(e1) / a.steps
    log(f"[bench] timed {a.steps} steps in {wall:.3f} s")

    # GPU-side launch duration: the same K back-to-back launches, queued
    # behind a ~0.35 ms copy so that the host has enqueued them all before
    # the first one starts. Microsecond-scale kernels are otherwise timed at
    # the host's submission rate (Python + launch API), not the GPU's.
    prime_n = 1 << 27
    pa, pb = kh.Buffer(4 * prime_n), kh.Buffer(4 * prime_n)
    for c in cases:
        e0, e1 = ev[c.name]
        kh.roofline_copy(pa, pb, prime_n, stream)
        e0.record(stream)
        for i in range(a.steps):
            c.launch(c.sets[(a.warmup + i) % len(c.sets)], stream)
        e1.record(stream)
        e1.synchronize()
        c.ms = [e0.elapsed_ms(e1) / a.steps]
    pa.free()
    pb.free()

    ceilings = None
    if not a.no_ceilings:
        ceilings = measure_ceilings(kh, stream)
        log(f"[bench] measured ceilings: triad {ceilings['hbm_triad_gbps']:.0f} GB/s, copy "
            f"{ceilings['hbm_copy_gbps']:.0f} GB/s, fp32 MFMA {ceilings['fp32_mfma_tflops']:.1f} TFLOP/s")

    kernels = {}
    for c in cases:
        ms = float(np.mean(c.ms))
        rate = c.work / (ms * 1e-3) / (1e12 if c.unit == "TFLOP/s" else 1e9)
        peak = FP32_MFMA_PEAK_TFLOPS if c.bound == "mfma" else HBM_PEAK_GBPS
        rate_host = c.work / (c.ms_host * 1e-3) / (1e12 if c.unit == "TFLOP/s" else 1e9)
        kernels[c.name] = {"config": c.config, "ms_mean": ms, "ms_host_paced": c.ms_host,
                           "rate": rate, "rate_host_paced": rate_host, "unit": c.unit,
                           "bound": c.bound, "peak": peak, "frac": rate / peak,
                           "algorithmic_work_per_launch": c.work, "buffer_sets": len(c.sets)}
        if ceilings:
            meas = ceilings["fp32_mfma_tflops"] if c.bound == "mfma" else ceilings["hbm_triad_gbps"]
            kernels[c.name]["measured_ceiling"] = meas
            kernels[c.name]["frac_of_measured"] = rate / meas
        if c.name in PMC_TRAFFIC_BYTES:
            kernels[c.name]["traffic_bytes_pmc"] = PMC_TRAFFIC_BYTES[c.name]
        if c.traffic_note:
            kernels[c.name]["note"] = c.traffic_note
        log(f"[bench] {c.name:10s} {ms:9.4f} ms  {rate:9.1f} {c.unit}  ({100 * rate / peak:5.1f}% of peak"
            + (f", {100 * kernels[c.name]['frac_of_measured']:5.1f}% of measured)" if ceilings else ")"))

    head = "gemm" if "gemm" in kernels else (cases[0].name if cases else None)
    hk = kernels.get(head, {})
    out = {
        "metric": METRIC,
        "value": hk.get("rate"),
        "unit": hk.get("unit", "TFLOP/s"),
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": wall * 1e3 / max(1, a.steps),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"kernel.h seven templates at BASELINE sizes; value = {head} "
                               "(gemm m=n=k=8192 fp32); per-kernel rates under 'kernels'",
                   "gemm": "m=n=k=8192", "softmax": "rows=4096,cols=1024", "scan": "n=2^26",
                   "vecadd": "n=2^24", "layernorm": "rows=4096,cols=1024", "fused_gelu": "n=2^26",
                   "attention": "batch=4,heads=16,seq=4096,head_dim=64",
                   "buffer_rotation": not a.no_rotate},
        "roofline": None if not hk else {
            "bound": hk["bound"], "achieved": hk["rate"], "peak": hk["peak"],
            "unit": hk["unit"], "frac": hk["frac"], "traffic": PMC_TRAFFIC_BYTES.get(head), "kernel": head},
        "kernels": kernels,
        "measured_ceilings": ceilings,
        "device": {"name": info["name"], "arch": info["arch"], "cu_count": info["cu_count"]},
    }
    if not a.no_cpu:
        log("[bench] cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline(a.cpu_budget)
        log(f"[bench] cpu baseline {out['cpu_baseline']['value']:.4f} TFLOP/s")
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
