#!/usr/bin/env python3
"""Benchmark of the kernel.h seven-template hot path on one MI355X.

One step = one pass of the suite the BASELINE metric is quoted on: the seven
templates at all thirteen BASELINE configurations. gemm 8192^3 is the
headline `value` (fp32 TFLOP/s); softmax 4096x1024 and scan 2^26 are the
metric's HBM rows; vecadd 2^24, layernorm 4096x1024, fused_gelu 2^22 and
2^26, scan 10^6, gemm 512^3 / 2048^3 / 8192x8192x256 and attention b4 h16 d64
at seq 1024 and 4096 complete it, each reported under "kernels". Inputs are
synthetic (seeded numpy generators of the BASELINE distributions), resident
in HBM before the timed region; every launch goes through the khrt C-ABI
(hipModuleLaunchKernel on the embedded gfx950 code objects).

Timing: W untimed warmup steps, then K timed steps bracketed by device
synchronisation. Per kernel, HIP events recorded on the launch stream around
its K back-to-back launches give the average launch duration. Working sets
smaller than 1 GiB rotate over several buffer sets so every launch reads
from HBM rather than the 256 MB Infinity Cache.

Roofline: `achieved` = algorithmic bytes (or FLOPs) per launch / average
launch duration; `peak` = MI355X published peak (HBM 8 TB/s; fp32 MFMA
157.3 TFLOP/s). The measured HBM ceiling of a kernel is the best of copy and
triad streams of 2^28 floats (2 and 3 GiB) and at that kernel's own bytes
per launch (rotated the same way), each with the product's streaming geometry and with a
32-workgroups-per-CU grid. The CPU baseline times the oracle's fp64
references on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import struct
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "kernel.h_amd"))

import numpy as np  # noqa: E402

HBM_PEAK_GBPS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
ROTATE_BYTES = 1 << 30  # rotate buffer sets until the working set exceeds 1 GiB

METRIC = "GEMM-8192 fp32 TFLOPS + softmax/scan HBM GB/s, % of MI355X roofline"

# HBM bytes per launch of every configuration, from two rocprofv3 --pmc passes
# (FETCH_SIZE x 2.000, WRITE_SIZE x 1.000: the factors a copy kernel of known
# size reads) over `bench.py --steps 2 --warmup 1 --no-cpu --no-ceilings` with
# its buffer rotation (working sets past 1 GiB), recorded in
# profiles/templates_baseline_sizes_hbm_traffic.md. Constants of that profile
# (median dispatch), not measured by the run that reports them.
PMC_TRAFFIC_BYTES = {
    "vecadd": 201358270, "softmax": 33658314, "layernorm": 33720774, "scan": 539174466, "scan_1e6": 8198139,
    "fused_gelu": 536929788, "fused_gelu_2^22": 33632843, "gemm": 3636852993, "gemm_8192x8192x256": 371314749, "gemm_2048": 117641828,
    "gemm_512": 10544554, "attention": 268738094, "attention_s1024": 67421693,
}
PMC_TRAFFIC_SOURCE = "profiles/templates_baseline_sizes_hbm_traffic.md (constant, not measured by this run)"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def u24(rng, n, lo, hi):
    """Uniform on the 2^-24 grid, lo + (hi-lo) u, rounded to fp32."""
    u = rng.integers(0, 1 << 24, n, dtype=np.int64).astype(np.float64) / float(1 << 24)
    return (lo + (hi - lo) * u).astype(np.float32)


def normal(rng, n, sd):
    return (rng.standard_normal(n) * sd).astype(np.float32)


class Case:
    """One template at one BASELINE configuration. `host` makes the seeded
    input arrays once; every buffer set gets its own device copies of them
    (plus its own outputs), so rotated launches read distinct memory."""

    def __init__(self, name, config, work, unit, bound, host, device, launch, note="", gemm_shape=None):
        self.name, self.config, self.work, self.unit, self.bound = name, config, work, unit, bound
        self.host, self.device, self.launch, self.note = host, device, launch, note
        self.gemm_shape = gemm_shape  # (m, n, k) for the vendor comparison leg
        self.sets = []
        self.ms = []


def make_cases(kh, rng, only):
    up = lambda a: kh.Buffer.from_array(a)
    out = lambda count: kh.Buffer(4 * count)
    cases = []

    def add(c):
        if only is None or c.name in only:
            cases.append(c)

    n = 1 << 24
    add(Case("vecadd", "n=2^24 fp32, a,b ~ U[-1,1]", 12.0 * n, "GB/s", "hbm",
             lambda: (u24(rng, n, -1, 1), u24(rng, n, -1, 1)),
             lambda h: (up(h[0]), up(h[1]), out(n)),
             lambda s, st: kh.vecadd(s[0], s[1], s[2], n, st)))

    R, C = 4096, 1024
    add(Case("softmax", "4096x1024 fp32, x ~ N(0, 4^2)", 8.0 * R * C, "GB/s", "hbm",
             lambda: (normal(rng, R * C, 4.0),),
             lambda h: (up(h[0]), out(R * C)),
             lambda s, st: kh.softmax(s[0], s[1], R, C, st)))

    add(Case("layernorm", "4096x1024 fp32, eps 1e-5, x ~ N(0, 4^2), gamma U[0.5,1.5], beta U[-0.1,0.1]",
             8.0 * R * C + 8.0 * C, "GB/s", "hbm",
             lambda: (normal(rng, R * C, 4.0), u24(rng, C, 0.5, 1.5), u24(rng, C, -0.1, 0.1)),
             lambda h: (up(h[0]), up(h[1]), up(h[2]), out(R * C)),
             lambda s, st: kh.layernorm(s[0], s[1], s[2], s[3], R, C, st)))

    def scan_case(name, ns, label):
        T = kh.scan_workspace_floats(ns)
        # One look-back workspace (totals_hi, totals_lo) per configuration,
        # reused by every call as a caller's workspace is; x and y rotate. A
        # fresh workspace per call would time the one-time header claim
        # (compare-and-swap, re-sign) on every launch.
        ws = []

        def device(h):
            if not ws:
                ws.extend((out(T), out(T)))
            return (up(h[0]), out(ns), ws[0], ws[1])
        return Case(name, f"inclusive n={label} fp32, x ~ U[0,1) on the 2^-24 grid", 8.0 * ns, "GB/s", "hbm",
                    lambda: (u24(rng, ns, 0, 1),), device,
                    lambda s, st: kh.scan(s[0], s[1], None, s[2], s[3], ns, st))

    add(scan_case("scan", 1 << 26, "2^26"))
    add(scan_case("scan_1e6", 1000000, "10^6"))

    def gelu_case(name, ng, label):
        return Case(name, f"n={label} fp32, x ~ N(0,1); out = gelu_tanh(1.5x+0.5)", 8.0 * ng, "GB/s", "hbm",
                    lambda: (normal(rng, ng, 1.0),),
                    lambda h: (up(h[0]), out(ng)),
                    lambda s, st: kh.fused_gelu(s[0], None, s[1], ng, st),
                    "reference formula counts 12 B/elem (metrics.cpp:36-38); 8 B/elem are moved")

    add(gelu_case("fused_gelu", 1 << 26, "2^26"))
    add(gelu_case("fused_gelu_2^22", 1 << 22, "2^22"))

    def gemm_case(name, m, nn, k):
        return Case(name, f"C=A*B fp32 row-major, m={m} n={nn} k={k}, A,B ~ U[-1,1]", 2.0 * m * nn * k,
                    "TFLOP/s", "mfma",
                    lambda: (u24(rng, m * k, -1, 1), u24(rng, k * nn, -1, 1)),
                    lambda h: (up(h[0]), up(h[1]), out(m * nn)),
                    lambda s, st: kh.gemm(s[0], s[1], s[2], m, nn, k, st), gemm_shape=(m, nn, k))

    add(gemm_case("gemm", 8192, 8192, 8192))
    add(gemm_case("gemm_512", 512, 512, 512))
    add(gemm_case("gemm_2048", 2048, 2048, 2048))
    add(gemm_case("gemm_8192x8192x256", 8192, 8192, 256))

    def attention_case(name, b, h, s_, d=64):
        e = b * h * s_ * d
        return Case(name, f"non-causal b={b} h={h} s={s_} d={d} fp32, Q,K,V ~ N(0,1)", 4.0 * b * h * s_ * s_ * d,
                    "TFLOP/s", "mfma",
                    lambda: tuple(normal(rng, e, 1.0) for _ in range(3)),
                    lambda hh: (up(hh[0]), up(hh[1]), up(hh[2]), out(e)),
                    lambda s, st: kh.attention(s[0], s[1], s[2], s[3], b, h, s_, d, st))

    add(attention_case("attention", 4, 16, 4096))
    add(attention_case("attention_s1024", 4, 16, 1024))
    return cases


def available(kh, name):
    try:
        kh.code_object(name.split("_")[0] if name.startswith(("gemm", "scan", "attention")) else
                       "fused_gelu" if name.startswith("fused_gelu") else name)
        return True
    except kh.KhrtError:
        return False


def set_bytes(sets):
    return sum(b.nbytes for b in sets)


def rotation_count(bytes_per_set, cap=1024):
    """Buffer sets it takes to exceed ROTATE_BYTES (at most cap)."""
    return max(1, min(cap, -(-ROTATE_BYTES // max(1, int(bytes_per_set)))))


def issue_ms(launches, sync):
    """Host time to issue `launches` back to back (an untimed pass; `sync`
    then waits for them)."""
    t0 = time.perf_counter()
    for f in launches:
        f()
    t1 = time.perf_counter()
    sync()
    return (t1 - t0) * 1e3


def prime_for(prime, stream, host_ms):
    """Queues enough primer copies (~0.35 ms each) ahead of a sequence whose
    launches take the host `host_ms` to issue: the host then enqueues the
    whole sequence before its first launch starts, so events around it time
    the GPU, not the host's submission rate."""
    for _ in range(max(1, -(-int(1.5 * host_ms * 1000) // 350))):
        prime(stream)


def time_queued(kh, stream, launches, prime):
    """Average GPU duration of `launches` (callables, issued back to back)
    queued behind primer copies that outlast the host's time to issue them
    (measured in an untimed pass first): microsecond kernels are timed at
    the GPU's rate, not the host's submission rate."""
    e0, e1 = kh.Event(), kh.Event()
    host = issue_ms(launches, stream.synchronize)
    prime_for(prime, stream, host)
    e0.record(stream)
    for f in launches:
        f()
    e1.record(stream)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / len(launches)
    e0.destroy()
    e1.destroy()
    return ms


def measure_ceilings(kh, stream, hbm_cases, prime, steps):
    """Measured roofline denominators.

    HBM: plain copy (8 B/float) and triad (12 B/float) streams, the
    reference's roofline_triad pattern (bench/refs/roofline.hip:22-30, 2^28
    floats: 2 GiB per copy launch, 3 GiB per triad launch, beyond the
    256 MB MALL) plus copies and triads
    of exactly each HBM kernel's bytes per launch, rotated like that
    kernel's buffers. Each runs under two geometries: the product streaming
    kernels' (one unrolled step per thread, ceil(n/4/1024) workgroups of
    256) and 32 grid-strided workgroups per CU, each the best of five
    sequences. A kernel's ceiling is the best of the 2^28-float streams and
    its own-size streams.

    fp32 MFMA: independent chains of each fp32 MFMA shape (8 of 32x32x2 or
    16 of 16x16x4 per wave), two waves per SIMD, ~3.5 ms per launch (shorter
    launches under-measure it, as the clock has not settled and launch gaps
    count); the best of three sequences of ten launches, the faster shape."""
    co = os.path.join(REPO, "kernel.h_amd", "build", "co", "roofline.hsaco")
    with open(co, "rb") as f:
        mod = kh.GpuModule(f.read())
    fn = {"copy": mod.get_function("roofline_copy"), "triad": mod.get_function("roofline_triad")}
    cu = kh.device_info()["cu_count"]

    def grids(n):
        return {"product": max(1, -(-(n // 4) // 1024)), "32/CU": 32 * cu}

    def stream_rate(kind, n, sets, grid, reps):
        def launch(bufs):
            args = kh.LaunchArgs()
            for b in bufs:
                args.add_memref(b, [n])
            return lambda: kh.launch_raw(fn[kind], (grid, 1, 1), (256, 1, 1), args, stream)
        calls = [launch(sets[i % len(sets)]) for i in range(reps)]
        calls[0]()
        # Best of five sequences: a ceiling is the most the pattern reached,
        # not one sample of it (the kernels' own rates are means).
        ms = min(time_queued(kh, stream, calls, prime) for _ in range(5))
        return (12.0 if kind == "triad" else 8.0) * n / (ms * 1e-3) / 1e9

    def streams(n, reps, rotate):
        per = {"copy": 2, "triad": 3}
        best, rows = 0.0, []
        for kind in ("copy", "triad"):
            nn = n["copy" if kind == "copy" else "triad"] if isinstance(n, dict) else n
            nn = max(4, nn - nn % 4)
            count = rotation_count(4 * nn * per[kind]) if rotate else 1
            sets = [tuple(kh.Buffer(4 * nn) for _ in range(per[kind])) for _ in range(count)]
            for s_ in sets:
                s_[0].fill(1.0, stream)
                if kind == "triad":
                    s_[1].fill(2.0, stream)
            for gname, g in grids(nn).items():
                r = stream_rate(kind, nn, sets, g, reps)
                rows.append({"kernel": kind, "floats": nn, "bytes": (12 if kind == "triad" else 8) * nn,
                             "grid": gname, "buffer_sets": len(sets), "gbps": r})
                best = max(best, r)
            for s_ in sets:
                for b in s_:
                    b.free()
        return best, rows

    big_best, big_rows = streams(1 << 28, 5, rotate=False)
    per_case = {}
    for c in hbm_cases:
        # As many launches per sequence as the kernel's own measurement.
        best, rows = streams({"copy": int(c.work // 8), "triad": int(c.work // 12)},
                             getattr(c, "gpu_launches", steps), rotate=True)
        per_case[c.name] = {"gbps": max(big_best, best), "own_size_best": best, "streams": rows}

    # Both fp32 MFMA shapes, ~3.5 ms launches, ten per sequence; the best of
    # three sequences each (clocks settle over the first launches).
    blocks, iters = cu * 2, 8192
    out = kh.Buffer(4 * blocks * 256)
    args16 = kh.LaunchArgs().add_memref(out, [blocks * 256]).add_scalar_bytes(struct.pack("<q", iters))
    mfma16 = mod.get_function("roofline_mfma16")
    runs = {"v_mfma_f32_32x32x2f32": (float(blocks) * 4 * iters * 8 * 32 * 32 * 2 * 2,
                                      lambda: kh.roofline_mfma(out, blocks, iters, stream)),
            "v_mfma_f32_16x16x4f32": (float(blocks) * 4 * iters * 16 * 16 * 16 * 4 * 2,
                                      lambda: kh.launch_raw(mfma16, (blocks, 1, 1), (256, 1, 1), args16, stream))}
    mfma_rates = {}
    for name, (flops, call) in runs.items():
        call()
        best = min(time_queued(kh, stream, [call] * 10, prime) for _ in range(3))
        mfma_rates[name] = flops / (best * 1e-3) / 1e12
    out.free()
    return {"hbm_2e28_floats_best_gbps": big_best, "hbm_2e28_floats_streams": big_rows,
            "hbm_2e28_floats_note": "copy 2^28 floats (2 GiB per launch) and triad 2^28 floats (3 GiB)",
            "hbm_per_kernel": per_case,
            "fp32_mfma_tflops": max(mfma_rates.values()), "fp32_mfma_by_instruction": mfma_rates,
            "mfma_config": f"{blocks} workgroups x 4 waves x {iters} rounds of independent chains "
                           "(8 of 32x32x2 or 16 of 16x16x4 per wave), best of 3 sequences of 10 launches"}


def _median_runs(fn, runs=3, long_s=10.0):
    """Median of `runs` timed calls of fn() (seconds), or the first alone
    when it ran longer than long_s."""
    times = []
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
        if times[0] > long_s:
            break
    return float(np.median(times)), len(times)


def cpu_baseline(budget_s: float):
    """The oracle's fp64 references (CPU restatements of the reference's
    e2e checks) timed on this host, built for its widest x86-64 level (the
    stand-in for -march=native), on all cores (OpenMP, the core count from
    sched_getaffinity) and on one core. Each rate is the median of 3 runs (1
    when a run exceeds 10 s). The headline, in `value`'s unit, is the GEMM
    reference (e2e_gemm_test.cpp:92-110) on a row sample of the 8192^3
    problem; `other_kernels` holds every other reference at its BASELINE
    configuration: vecadd's fp64 sum, softmax_reference_row, layernorm's
    reference_row, gelu_reference, the serial scan prefix (one core: it is a
    recurrence) and attention_reference_row on a row sample of b4 h16 s4096
    (rates of samples are extrapolated to the whole problem, so labelled)."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    isa = O.host_isa()
    O.use_isa(isa)
    cores = len(os.sched_getaffinity(0))
    M = 8192
    rng = np.random.default_rng(7)
    A = u24(rng, M * M, -1, 1)
    B = u24(rng, M * M, -1, 1)

    def sample_size(run, threads, target, first):
        # Grows a sample (rows or elements) until one run takes >= 50 ms,
        # then scales it to take about `target` seconds.
        O.set_threads(threads)
        size = first
        while True:
            t = time.perf_counter()
            run(size)
            dt = time.perf_counter() - t
            if dt >= 0.05:
                break
            size *= 4
        return max(first, int(size * target / dt))

    def gemm_rate(threads, share):
        rows = min(M, sample_size(lambda r: O.ref_gemm(A, B, M, M, M, row0=0, nrows=min(M, r)), threads,
                                  share * budget_s / 3, max(threads, 2)))
        med, k = _median_runs(lambda: O.ref_gemm(A, B, M, M, M, row0=0, nrows=rows))
        return 2.0 * rows * M * M / med / 1e12, rows, med, k

    tf_all, rows_all, s_all, k_all = gemm_rate(cores, 0.35)
    tf_one, rows_one, s_one, k_one = gemm_rate(1, 0.2)
    del A, B

    def both(fn, work):
        # fn() timed on all cores and on one: work / median seconds.
        out = {}
        for label, threads in (("all_cores", cores), ("single_thread", 1)):
            O.set_threads(threads)
            med, _ = _median_runs(fn)
            out[label] = work / med / 1e9
        return out

    other = {}
    n = 1 << 24
    va, vb = u24(rng, n, -1, 1), u24(rng, n, -1, 1)
    other["vecadd_2^24_gbps"] = both(lambda: O.ref_vecadd(va, vb), 12.0 * n)
    del va, vb
    R, C = 4096, 1024
    x = normal(rng, R * C, 4.0)
    other["softmax_4096x1024_gbps"] = both(lambda: O.ref_softmax(x, R, C), 8.0 * R * C)
    g, bt = u24(rng, C, 0.5, 1.5), u24(rng, C, -0.1, 0.1)
    other["layernorm_4096x1024_gbps"] = both(lambda: O.ref_layernorm(x, g, bt, R, C), 8.0 * R * C + 8.0 * C)
    ng = 1 << 22
    xg = normal(rng, ng, 1.0)
    other["fused_gelu_2^22_gbps"] = both(lambda: O.ref_gelu(xg), 8.0 * ng)
    xs = u24(rng, 1 << 26, 0, 1)
    O.set_threads(1)
    sc_one, _ = _median_runs(lambda: O.ref_scan(xs))
    other["scan_2^26_gbps_single_thread"] = 8.0 * xs.size / sc_one / 1e9
    del xs
    # attention b4 h16 s4096 d64: a sample of query rows spread over the 64
    # slices; rate = 4 s d FLOP per row (4 b h s^2 d over b h s rows).
    b, h, s_, d = 4, 16, 4096, 64
    Q, K, V = (normal(rng, b * h * s_ * d, 1.0) for _ in range(3))
    att = {}
    for label, threads, share in (("all_cores", cores, 0.06), ("single_thread", 1, 0.04)):
        def rows_run(r):
            idx = np.arange(r, dtype=np.int64) * 7919 % (b * h * s_)
            O.ref_attention_rows(Q, K, V, s_, d, idx // s_, idx % s_)
        rows = min(b * h * s_, sample_size(rows_run, threads, share * budget_s / 3, max(threads, 4)))
        med, _ = _median_runs(lambda: rows_run(rows))
        att[label] = 4.0 * s_ * d * rows / med / 1e12
        att[label + "_rows"] = rows
    other["attention_b4h16s4096_tflops_extrapolated"] = att
    del Q, K, V
    other["note"] = ("fp64 references, same input distributions as the GPU rows; GB/s counts the kernel's "
                     "algorithmic bytes (fused_gelu 8 B per element: tmp is dead); the scan prefix is serial; "
                     "medians of 3 runs; attention on a row sample, extrapolated")
    O.set_threads(cores)
    return {"value": tf_all, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"fp64 rank-1 GEMM reference (oracle kho_ref_gemm, built for {isa}): rows 0..{rows_all} of "
                      f"the 8192^3 problem on {cores} threads, median of {k_all} runs of {s_all:.2f} s, "
                      "extrapolated to the whole problem",
            "single_thread": {"value": tf_one, "unit": "TFLOP/s", "cores": 1,
                              "sample": f"{rows_one} rows, median of {k_one} runs of {s_one:.2f} s"},
            "other_kernels": other,
            "isa": isa}


def measure_vendor_gemm(torch, gemm_cases, steps, prime):
    """The vendor fp32 GEMM (torch.mm: hipBLASLt or rocBLAS, TF32 off) on each
    GEMM case's shape, under this bench's own conditions: as many rotated
    buffer sets as the case, U[-1,1] inputs, K back-to-back launches between
    two events on torch's stream (as many as this build's own measurement of
    the case), queued behind primer copies that outlast the host's time to
    issue them (torch.mm's per-call host cost exceeds a 512^3 kernel), so
    the rate is the vendor kernel's. A reference point for the same shapes,
    not part of this build's result."""
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    res = {}
    for c in gemm_cases:
        m, n, k = c.gemm_shape
        gen = torch.Generator(device=dev).manual_seed(20261201)
        sets = [(torch.rand(m, k, device=dev, generator=gen) * 2 - 1, torch.rand(k, n, device=dev, generator=gen) * 2 - 1,
                 torch.empty(m, n, device=dev)) for _ in range(len(c.sets))]
        st = torch.cuda.current_stream()
        for i in range(3):
            x, y, z = sets[i % len(sets)]
            torch.mm(x, y, out=z)
        best = None
        count = c.gpu_launches  # the same number of launches as this build's measurement
        calls = [lambda i=i: torch.mm(sets[i % len(sets)][0], sets[i % len(sets)][1], out=sets[i % len(sets)][2])
                 for i in range(count)]
        host = issue_ms(calls, torch.cuda.synchronize)
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            prime_for(prime, st.cuda_stream, host)
            e0.record(st)
            for i in range(count):
                x, y, z = sets[i % len(sets)]
                torch.mm(x, y, out=z)
            e1.record(st)
            e1.synchronize()
            ms = e0.elapsed_time(e1) / count
            best = ms if best is None else min(best, ms)
        res[c.name] = {"ms": best, "rate": 2.0 * m * n * k / (best * 1e-3) / 1e12, "unit": "TFLOP/s",
                       "buffer_sets": len(sets), "library": "torch.mm (hipBLASLt/rocBLAS), tf32 off",
                       "launches_averaged": count, "host_issue_ms": host,
                       "timing": "best of 3 sequences, GPU-paced (queued behind primers that outlast their issue)"}
        del sets
        torch.cuda.empty_cache()
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--kernels", default="", help="comma list to restrict the suite")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-rotate", action="store_true", help="reuse one buffer set (cache-warm)")
    ap.add_argument("--no-ceilings", action="store_true", help="skip the measured roofline microbenchmarks")
    ap.add_argument("--no-vendor", action="store_true", help="skip the vendor GEMM comparison (torch.mm)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}); "
              "multi-GPU runs are out of scope", file=sys.stderr)
        return 2

    torch = None
    if not a.no_vendor:
        try:
            import torch  # noqa: F811  (vendor GEMM comparison only)
            if not torch.cuda.is_available():
                torch = None
        except Exception:
            torch = None
    import kernelh as kh
    kh.init_device(0)
    info = kh.device_info()
    log(f"[bench] device {info['name']} {info['arch']} cu={info['cu_count']}")
    rng = np.random.default_rng(20261201)
    only = set(a.kernels.split(",")) if a.kernels else None
    cases = [c for c in make_cases(kh, rng, only) if available(kh, c.name)]
    stream = kh.Stream()

    for c in cases:
        h = c.host()
        first = c.device(h)
        count = 1 if a.no_rotate else rotation_count(set_bytes(first))
        c.sets = [first] + [c.device(h) for _ in range(count - 1)]
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

    # GPU-side launch duration: back-to-back launches over the same buffer
    # sets, queued behind a ~0.35 ms copy so that the host has enqueued them
    # all before the first one starts (time_queued).
    prime_n = 1 << 27
    prime_bufs = (kh.Buffer(4 * prime_n), kh.Buffer(4 * prime_n))
    prime = lambda st: kh.roofline_copy(prime_bufs[0], prime_bufs[1], prime_n, st)
    # At least ~0.4 ms of launches per kernel (from the timed region's
    # duration), so the first launches after the primer do not dominate a
    # microsecond kernel's average: ~57 launches of a 7 us kernel.
    for c in cases:
        count = max(a.steps, min(256, int(0.4 / max(c.ms_host, 1e-4)) + 1))
        c.gpu_launches = count
        c.ms = [time_queued(kh, stream, [lambda c=c, i=i: c.launch(c.sets[(a.warmup + i) % len(c.sets)], stream)
                                         for i in range(count)], prime)]

    ceilings = None
    if not a.no_ceilings:
        ceilings = measure_ceilings(kh, stream, [c for c in cases if c.bound == "hbm"], prime, a.steps)
        log(f"[bench] measured ceilings: HBM streams of 2^28 floats {ceilings['hbm_2e28_floats_best_gbps']:.0f} GB/s, "
            f"fp32 MFMA {ceilings['fp32_mfma_tflops']:.1f} TFLOP/s")
    vendor = {}
    gemm_cases = [c for c in cases if c.gemm_shape]
    if torch is not None and gemm_cases:
        vendor = measure_vendor_gemm(torch, gemm_cases, a.steps, prime)
        log("[bench] vendor fp32 GEMM: " + ", ".join(f"{k} {v['rate']:.1f}" for k, v in vendor.items()))
    prime_bufs[0].free()
    prime_bufs[1].free()

    kernels = {}
    for c in cases:
        ms = float(np.mean(c.ms))
        rate = c.work / (ms * 1e-3) / (1e12 if c.unit == "TFLOP/s" else 1e9)
        peak = FP32_MFMA_PEAK_TFLOPS if c.bound == "mfma" else HBM_PEAK_GBPS
        rate_host = c.work / (c.ms_host * 1e-3) / (1e12 if c.unit == "TFLOP/s" else 1e9)
        k = {"config": c.config, "ms_mean": ms, "ms_host_paced": c.ms_host,
             "rate": rate, "rate_host_paced": rate_host, "unit": c.unit,
             "bound": c.bound, "peak": peak, "frac": rate / peak,
             "algorithmic_work_per_launch": c.work, "buffer_sets": len(c.sets), "gpu_launches_averaged": c.gpu_launches}
        if ceilings:
            if c.bound == "mfma":
                k["measured_ceiling"] = ceilings["fp32_mfma_tflops"]
                k["measured_ceiling_source"] = "fp32 MFMA microbenchmark"
            else:
                pc = ceilings["hbm_per_kernel"][c.name]
                k["measured_ceiling"] = pc["gbps"]
                k["measured_ceiling_source"] = ("best of copy/triad streams of 2^28 floats (2 and 3 GiB) and at "
                                                "this kernel's "
                                                f"{int(c.work)} B per launch (own size best {pc['own_size_best']:.0f})")
            k["frac_of_measured"] = rate / k["measured_ceiling"]
        if c.name in PMC_TRAFFIC_BYTES:
            k["traffic_bytes_pmc"] = PMC_TRAFFIC_BYTES[c.name]
            k["traffic_source"] = PMC_TRAFFIC_SOURCE
        if c.note:
            k["note"] = c.note
        if c.name in vendor:
            k["vendor"] = dict(vendor[c.name], ratio=rate / vendor[c.name]["rate"])
        kernels[c.name] = k
        log(f"[bench] {c.name:20s} {ms:9.4f} ms  {rate:9.1f} {c.unit}  ({100 * rate / peak:5.1f}% of peak"
            + (f", {100 * k['frac_of_measured']:5.1f}% of measured)" if ceilings else ")"))

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
        "config": {"workload": f"kernel.h seven templates at all 13 BASELINE configurations; value = {head} "
                               "(gemm m=n=k=8192 fp32); per-kernel rates under 'kernels'",
                   "gemm": "m=n=k=8192; also 512^3, 2048^3, 8192x8192x256",
                   "softmax": "rows=4096,cols=1024", "scan": "n=2^26; also 10^6",
                   "vecadd": "n=2^24", "layernorm": "rows=4096,cols=1024", "fused_gelu": "n=2^26; also 2^22",
                   "attention": "batch=4,heads=16,head_dim=64, seq=4096; also 1024",
                   "buffer_rotation": not a.no_rotate},
        "roofline": None if not hk else {
            "bound": hk["bound"], "achieved": hk["rate"], "peak": hk["peak"],
            "unit": hk["unit"], "frac": hk["frac"], "traffic": PMC_TRAFFIC_BYTES.get(head), "kernel": head,
            "traffic_source": PMC_TRAFFIC_SOURCE if head in PMC_TRAFFIC_BYTES else None},
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
