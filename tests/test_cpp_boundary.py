"""The C++ surfaces over the C-ABI.

- include/khrt.hpp: RAII DeviceContext / Buffer / GpuModule / LaunchArgs /
  KernelLaunch / EventTimer with their own Result<T>, in the shapes of the
  reference's runtime classes (include/kernelh/runtime/*.hpp).
- kernel.h_amd/integration/backend_khrt.cpp: the reference's Backend
  (backend.hpp:56-96) implemented over khrt, compiled here against a
  restatement of backend.hpp, and shown verbatim in the integration guide.

On the CPU the check programs run their error-path and packing checks; on
the GPU they launch vecadd and scan through those interfaces and compare
bit-exactly. The programs are built in-tree by kernel.h_amd/build.py.
"""
import os
import subprocess

import pytest

import kernelh as kh

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RAII = os.path.join(kh.BUILD, "khrt_raii_check")
BACKEND = os.path.join(kh.BUILD, "khrt_backend_check")
BINDING = os.path.join(REPO, "kernel.h_amd", "integration", "backend_khrt.cpp")
RESTATED = os.path.join(REPO, "tests", "cpp", "restated")


def run(exe, mode, timeout=120):
    assert os.path.exists(exe), f"{exe} is not built (python kernel.h_amd/build.py)"
    r = subprocess.run([exe, mode], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=timeout)
    return r.returncode, r.stdout


@pytest.mark.parametrize("exe,name", [(RAII, "raii_check"), (BACKEND, "backend_check")], ids=["raii", "backend"])
def test_check_programs_cpu(exe, name):
    if kh.device_count() > 0:
        pytest.skip("a device is visible: the gpu mode covers these checks")
    rc, out = run(exe, "cpu")
    assert rc == 0, out
    assert out.splitlines()[-1].startswith(f"{name} cpu ok")


def test_backend_binding_compiles_against_restated_interface(tmp_path):
    """The binding, as a maintainer would add it to the reference tree, builds
    and links against libkhrt.so with the restated backend.hpp, and its
    error paths behave without a device."""
    exe = tmp_path / "backend_check"
    r = subprocess.run(["g++", "-std=c++20", "-Wall", "-Wextra", "-Werror", f"-I{REPO}/include", f"-I{RESTATED}",
                        "-o", str(exe), os.path.join(REPO, "tests", "cpp", "backend_check.cpp"), BINDING,
                        f"-L{kh.BUILD}", "-lkhrt", f"-Wl,-rpath,{kh.BUILD}"],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    assert r.returncode == 0, r.stdout
    if kh.device_count() == 0:
        rc, out = run(str(exe), "cpu")
        assert rc == 0, out


def test_raii_header_is_cxx17(tmp_path):
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-fsyntax-only", f"-I{REPO}/include",
                        os.path.join(REPO, "tests", "cpp", "raii_check.cpp")],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    assert r.returncode == 0, r.stdout


def test_integration_guide_shows_the_compiled_binding():
    with open(os.path.join(REPO, "INTEGRATION.md")) as f:
        guide = f.read()
    with open(BINDING) as f:
        src = f.read()
    assert "```cpp\n" + src + "```" in guide


@pytest.mark.gpu
@pytest.mark.parametrize("exe,name", [(RAII, "raii_check"), (BACKEND, "backend_check")], ids=["raii", "backend"])
def test_check_programs_gpu(dev, exe, name):
    print(f"[gpu-case] {name} gpu", flush=True)
    rc, out = run(exe, "gpu", timeout=100)
    assert rc == 0, out
    assert out.splitlines()[-1].startswith(f"{name} gpu ok"), out
