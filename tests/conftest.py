"""pytest configuration: the `gpu` marker, import paths, and build-on-demand.

Tests marked `gpu` need an MI355X (gfx950) and call the product only through
the khrt C-ABI (libkhrt.so). Everything else runs on the CPU: the oracle
against the reference's recipes and closed forms, and the host-side boundary
(descriptor packing, device limits, launch verifier, occupancy, library
exports, code objects).
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "kernel.h_amd"), os.path.join(REPO, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

_LIB = os.path.join(REPO, "kernel.h_amd", "build", "libkhrt.so")
_ORACLE = os.path.join(REPO, "oracle", "_build", "liboracle.so")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the khrt C-ABI")
    # Load what is built; build only when nothing is (e.g. a fresh checkout).
    if not os.path.exists(_LIB):
        sys.path.insert(0, os.path.join(REPO, "kernel.h_amd"))
        import build as _b  # kernel.h_amd/build.py
        _b.build()
    if not os.path.exists(_ORACLE):
        import oracle as _o
        _o.build()


@pytest.fixture(scope="session")
def dev():
    """Initialised device 0; fails (never skips) when no GPU is visible, so a
    GPU run cannot pass on a silently missing device."""
    import kernelh as kh
    n = kh.device_count()
    assert n >= 1, "no HIP device visible: gpu tests need an MI355X"
    kh.init_device(0)
    info = kh.device_info()
    print(f"\n[device] {info['name']} arch={info['arch']} cu={info['cu_count']} "
          f"lds={info['lds_bytes_per_workgroup']} wave={info['wavefront_size']}", flush=True)
    return info
