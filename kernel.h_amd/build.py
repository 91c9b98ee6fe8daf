"""Builds the gfx950 kernel.h runtime in-tree (no cmake/ninja needed).

Outputs under kernel.h_amd/build/:
  co/<name>.hsaco      bare-ELF gfx950 code objects (one per kernel source)
  co/<name>.isa        AMD assembly of those code objects (our own build)
  co/<name>.notes.json resource notes per kernel symbol
  gen/kh_embed.S       .incbin of every product code object
  gen/kh_resources.inc resource table compiled into the runtime
  gen/kh_cli_embed.S   .incbin of the CLI-only code objects (hipref)
  libkhrt.so           the C-ABI runtime (include/khrt.h)
  kernelh              the CLI (compile / bench / occupancy)
  khrt_raii_check, khrt_backend_check, co/mfma_probe.hsaco
                       test fixtures (sources under tests/)

Usage: python kernel.h_amd/build.py [-j N] [-v]
"""
from __future__ import annotations

import argparse
import json
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

import yaml

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
READELF = os.path.join(ROCM, "llvm", "bin", "llvm-readelf")
OBJDUMP = os.path.join(ROCM, "llvm", "bin", "llvm-objdump")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"

KDIR = os.path.join(HERE, "csrc", "kernels")
RDIR = os.path.join(HERE, "csrc", "runtime")
CLIDIR = os.path.join(HERE, "csrc", "cli")
BUILD = os.path.join(HERE, "build")
CO = os.path.join(BUILD, "co")
GEN = os.path.join(BUILD, "gen")
OBJ = os.path.join(BUILD, "obj")

# GEMM tune candidates: csrc/kernels/gemm_tune.hip compiled once per part of
# its list (gemm_tune_list.h, KH_GEMM_TUNE_PARTS = 4), so the parts compile
# in parallel. Embedded in the runtime: the launcher runs a candidate when a
# tune cache names it, and `kernelh tune` evaluates them through the runtime.
TUNE_PARTS = 4
VARIANTS = {f"gemm_tune{p}": ("gemm_tune", [f"-DKH_GEMM_TUNE_PART={p}"]) for p in range(TUNE_PARTS)}
# Product code objects embedded in libkhrt.so (order = kh_embed.S order).
PRODUCT = ["vecadd", "fused_gelu", "softmax", "layernorm", "scan", "gemm", "attention", "util", "roofline",
           *VARIANTS]
# Test fixtures, built here so that no GPU run compiles anything:
#   tests/fixtures/<name>.hip -> co/<name>.hsaco, loaded by tests through
#     khrt_module_load_data (never embedded in the runtime);
#   tests/cpp/<name>.cpp -> build/<name>, C++ programs over include/khrt.hpp
#     and over the reference-side Backend binding.
TDIR = os.path.join(REPO, "tests")
PROBES = ["mfma_probe"]
#   csrc/kernels/<base>.hip with test-only defines -> co/<name>.hsaco, also
#     loaded by tests only: scan with a short bounded wait, so that a test can
#     make its give-up paths run (every kernel still exits normally).
TEST_VARIANTS = {"scan_shortspin": ("scan", ["-DKH_SCAN_SPIN_LIMIT=2048"])}
CPP_CHECKS = {
    "khrt_raii_check": ["cpp/raii_check.cpp"],
    "khrt_backend_check": ["cpp/backend_check.cpp", "../kernel.h_amd/integration/backend_khrt.cpp"],
}
# CLI-only code objects, embedded in the kernelh executable: the bench
# comparators (csrc/cli/hipref.hip).
CLI_CODE_OBJECTS = {"hipref": "cli"}

DEVICE_FLAGS = [
    "-x", "hip", f"--offload-arch={ARCH}", "--cuda-device-only", "--no-gpu-bundle-output",
    "-O3", "-std=c++17", "-ffp-contract=fast",
    # No packed-fp32 instructions anywhere in this build.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", KDIR,
]
# Per-code-object additions. scan: the atomic optimizer rewrites the ticket
# atomicAdd into a wave-reduced form whose result is read back at once,
# which makes the wave wait for the atomic (and every older memory operation)
# right where it is issued; the plain atomic's result is first waited on at
# the barrier that publishes it.
EXTRA_DEVICE_FLAGS = {
    "scan": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}
HOST_FLAGS = [
    "-O2", "-g", "-fPIC", "-std=c++20", "-Wall", "-Wextra", "-fvisibility=hidden",
    "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{REPO}/include",
    f"-I{HERE}/csrc/include", f"-I{KDIR}", f"-I{GEN}",
]


def run(cmd, verbose=False, **kw):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, **kw)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out:
        print(out)
    return r.stdout


def compile_co(name: str, verbose: bool, srcdir: str = "") -> str:
    base, defs = VARIANTS.get(name) or TEST_VARIANTS.get(name) or (name, [])
    src = os.path.join(srcdir or KDIR, base + ".hip")
    out = os.path.join(CO, name + ".hsaco")
    run([HIPCC, *DEVICE_FLAGS, *EXTRA_DEVICE_FLAGS.get(base, []), *defs, "-c", src, "-o", out], verbose)
    isa = run([OBJDUMP, "-d", f"--mcpu={ARCH}", out])
    with open(os.path.join(CO, name + ".isa"), "w") as f:
        f.write(isa)
    notes = parse_notes(out)
    with open(os.path.join(CO, name + ".notes.json"), "w") as f:
        json.dump(notes, f, indent=1)
    return out


def parse_notes(path: str) -> list[dict]:
    text = run([READELF, "--notes", path])
    start = text.index("---")
    end = text.index("\n...", start)
    meta = yaml.safe_load(text[start:end])
    kernels = []
    for k in meta.get("amdhsa.kernels", []):
        kernels.append({
            "name": k[".name"],
            "vgpr_count": int(k.get(".vgpr_count", 0)),
            "agpr_count": int(k.get(".agpr_count", 0)),
            "sgpr_count": int(k.get(".sgpr_count", 0)),
            "lds_bytes": int(k.get(".group_segment_fixed_size", 0)),
            "private_segment_bytes": int(k.get(".private_segment_fixed_size", 0)),
            "wavefront_size": int(k.get(".wavefront_size", 64)),
            "max_flat_workgroup_size": int(k.get(".max_flat_workgroup_size", 0)),
            "kernarg_bytes": int(k.get(".kernarg_segment_size", 0)),
            # Explicit parameters only; hidden_* arguments (grid/block
            # counts) are appended and filled by the HIP runtime itself.
            "explicit_args": [int(a[".size"]) for a in k.get(".args", [])
                              if not str(a.get(".value_kind", "")).startswith("hidden_")],
            "vgpr_spill_count": int(k.get(".vgpr_spill_count", 0)),
            "sgpr_spill_count": int(k.get(".sgpr_spill_count", 0)),
        })
    return kernels


def write_embed(present: dict[str, str]) -> str:
    lines = ["/* Generated by kernel.h_amd/build.py: embedded gfx950 code objects. */",
             '\t.section .rodata.kh_co,"a",@progbits']
    for name in PRODUCT:
        lines += ["\t.p2align 12", f"\t.globl kh_co_{name}", f"\t.globl kh_co_{name}_end",
                  f"kh_co_{name}:"]
        if name in present:
            lines.append(f'\t.incbin "{present[name]}"')
        lines.append(f"kh_co_{name}_end:")
    lines += ["\t.byte 0", '\t.section .note.GNU-stack,"",@progbits', ""]
    path = os.path.join(GEN, "kh_embed.S")
    with open(path, "w") as f:
        f.write("\n".join(lines))
    return path


def write_resources(present: dict[str, str]) -> str:
    rows = []
    for name in PRODUCT:
        if name not in present:
            continue
        with open(os.path.join(CO, name + ".notes.json")) as f:
            for k in json.load(f):
                rows.append('{"%s", {%d, %d, %d, %d, %d, %d, %d}},' % (
                    k["name"], k["vgpr_count"], k["agpr_count"], k["sgpr_count"], k["lds_bytes"],
                    k["private_segment_bytes"], k["wavefront_size"], k["max_flat_workgroup_size"]))
    path = os.path.join(GEN, "kh_resources.inc")
    with open(path, "w") as f:
        f.write("// Generated by kernel.h_amd/build.py from the code-object notes.\n")
        f.write("\n".join(rows) + "\n")
    return path


def build(jobs: int = 8, verbose: bool = False) -> None:
    if os.path.isdir(BUILD):
        shutil.rmtree(BUILD)
    for d in (CO, GEN, OBJ):
        os.makedirs(d, exist_ok=True)

    srcs = [n for n in PRODUCT if os.path.exists(os.path.join(KDIR, VARIANTS.get(n, (n,))[0] + ".hip"))]
    fixture_dir = os.path.join(TDIR, "fixtures")
    probes = [n for n in PROBES if os.path.exists(os.path.join(fixture_dir, n + ".hip"))]
    cli_dirs = {n: (CLIDIR if d == "cli" else KDIR) for n, d in CLI_CODE_OBJECTS.items()}
    cli_cos = [n for n in CLI_CODE_OBJECTS if os.path.exists(os.path.join(cli_dirs[n], n + ".hip"))]
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        outs = dict(zip(srcs, ex.map(lambda n: compile_co(n, verbose), srcs)))
        list(ex.map(lambda n: compile_co(n, verbose, fixture_dir), probes))
        list(ex.map(lambda n: compile_co(n, verbose), TEST_VARIANTS))
        cli_outs = dict(zip(cli_cos, ex.map(lambda n: compile_co(n, verbose, cli_dirs[n]), cli_cos)))
    present = {n: p for n, p in outs.items() if n in PRODUCT}

    # Refuse spills into scratch in product kernels: they would silently
    # cost HBM bandwidth.
    for name in present:
        with open(os.path.join(CO, name + ".notes.json")) as f:
            for k in json.load(f):
                if k["private_segment_bytes"] > 0 or k["vgpr_spill_count"] > 0:
                    print(f"warning: {k['name']} uses {k['private_segment_bytes']} B of scratch "
                          f"({k['vgpr_spill_count']} VGPR spills)", file=sys.stderr)

    embed = write_embed(present)
    write_resources(present)

    # Runtime sources: plain C++ (host compiler) and HIP (hipcc, host code
    # plus the device variables they register with the HIP runtime).
    rt_srcs = sorted(os.path.join(RDIR, f) for f in os.listdir(RDIR) if f.endswith((".cpp", ".hip")))

    def cxx(src):
        obj = os.path.join(OBJ, os.path.basename(src) + ".o")
        if src.endswith(".hip"):
            run([HIPCC, "-x", "hip", f"--offload-arch={ARCH}", "-O2", "-fPIC", "-std=c++17",
                 "-fvisibility=hidden", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                 f"-I{REPO}/include", f"-I{HERE}/csrc/include", f"-I{KDIR}", "-c", src, "-o", obj], verbose)
        else:
            run([CXX, *HOST_FLAGS, "-c", src, "-o", obj], verbose)
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(cxx, rt_srcs))
    embed_obj = os.path.join(OBJ, "kh_embed.o")
    run([CXX, "-c", embed, "-o", embed_obj], verbose)
    lib = os.path.join(BUILD, "libkhrt.so")
    run([CXX, "-shared", "-o", lib, *objs, embed_obj, f"-L{ROCM}/lib", "-lamdhip64",
         f"-Wl,-rpath,{ROCM}/lib", "-Wl,--no-undefined"], verbose)

    cli_srcs = sorted(os.path.join(CLIDIR, f) for f in os.listdir(CLIDIR) if f.endswith(".cpp")) \
        if os.path.isdir(CLIDIR) else []
    if cli_srcs:
        lines = ["/* Generated by kernel.h_amd/build.py: CLI comparator code objects. */",
                 '\t.section .rodata.kh_cli_co,"a",@progbits']
        for name in CLI_CODE_OBJECTS:
            lines += ["\t.p2align 12", f"\t.globl kh_cli_co_{name}", f"\t.globl kh_cli_co_{name}_end",
                      f"kh_cli_co_{name}:"]
            if name in cli_outs:
                lines.append(f'\t.incbin "{cli_outs[name]}"')
            lines.append(f"kh_cli_co_{name}_end:")
        lines += ["\t.byte 0", '\t.section .note.GNU-stack,"",@progbits', ""]
        cli_embed = os.path.join(GEN, "kh_cli_embed.S")
        with open(cli_embed, "w") as f:
            f.write("\n".join(lines))
        cli_embed_obj = os.path.join(OBJ, "kh_cli_embed.o")
        run([CXX, "-c", cli_embed, "-o", cli_embed_obj], verbose)
        run([CXX, *HOST_FLAGS, "-o", os.path.join(BUILD, "kernelh"), *cli_srcs, cli_embed_obj, f"-L{BUILD}",
             "-lkhrt", "-ldl", "-Wl,-rpath,$ORIGIN", f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib"],
            verbose)
    # The C++ check programs (test fixtures) over the installed interface:
    # include/ plus, for the Backend binding, tests/cpp/restated.
    for exe, parts in CPP_CHECKS.items():
        cpp = [os.path.normpath(os.path.join(TDIR, p)) for p in parts]
        if all(os.path.exists(p) for p in cpp):
            run([CXX, "-O1", "-g", "-std=c++20", "-Wall", "-Wextra", f"-I{REPO}/include",
                 f"-I{os.path.join(TDIR, 'cpp', 'restated')}", "-o", os.path.join(BUILD, exe), *cpp,
                 f"-L{BUILD}", "-lkhrt", "-Wl,-rpath,$ORIGIN"], verbose)
    if verbose:
        print("built", lib)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=8)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    build(a.j, a.v)
    return 0


if __name__ == "__main__":
    sys.exit(main())
