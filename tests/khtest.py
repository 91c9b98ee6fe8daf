"""Helpers for the GPU parity tests (imported by tests/test_gpu_*.py)."""
import sys

import numpy as np

import kernelh as kh


def say(msg: str) -> None:
    """Names the case before a GPU step, flushed, so a fault names its case."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def up(a) -> kh.Buffer:
    return kh.Buffer.from_array(np.ascontiguousarray(a, dtype=np.float32))


def empty(count: int, poison: float | None = float("nan")) -> kh.Buffer:
    """A float buffer pre-filled on the device (NaN by default) so an output
    element the kernel fails to write cannot pass a comparison by luck. The
    fill runs on the null stream, which does not order against the
    non-blocking streams kh.Stream creates, so it is waited for here."""
    b = kh.Buffer(max(1, count) * 4)
    if poison is not None:
        b.fill(poison)
        kh.synchronize()
    return b


def down(b: kh.Buffer, count: int) -> np.ndarray:
    kh.synchronize()
    return b.to_host(np.float32, count)
