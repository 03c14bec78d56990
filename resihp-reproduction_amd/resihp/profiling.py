"""Per-launch GPU timing of the library's kernels with HIP events.

``record()`` is a context manager: while it is active every GEMM and attention
launch made through :mod:`resihp.ops` is bracketed by two ``torch.cuda.Event``s
on the stream it is enqueued on (the current stream), labelled with the kernel
instantiation it selects and annotated with its algorithmic FLOPs.  After a
``torch.cuda.synchronize()``, ``summary()`` gives per-label launch counts, mean
duration and achieved TFLOP/s.  Inactive, it costs one attribute check per call.
"""

from __future__ import annotations

import contextlib

import torch

_active: list | None = None

LAYOUT_NAMES = {0: "NT", 1: "NN", 2: "TN"}
EPI_NAMES = {0: "none", 1: "gelu", 2: "gelu_grad"}


def active() -> bool:
    return _active is not None


@contextlib.contextmanager
def launch(label: str, flops: float):
    if _active is None:
        yield
        return
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    try:
        yield
    finally:
        end.record()
        _active.append((label, flops, start, end))


@contextlib.contextmanager
def record():
    global _active
    prev = _active
    _active = []
    try:
        yield _active
    finally:
        _active = prev


def summary(events) -> dict:
    """{label: {"launches", "mean_ms", "total_ms", "flops_per_launch", "tflops"}}."""
    out: dict = {}
    for label, flops, s, e in events:
        ms = s.elapsed_time(e)
        d = out.setdefault(label, {"launches": 0, "total_ms": 0.0, "flops": 0.0})
        d["launches"] += 1
        d["total_ms"] += ms
        d["flops"] += flops
    for d in out.values():
        d["mean_ms"] = d["total_ms"] / d["launches"]
        d["flops_per_launch"] = d["flops"] / d["launches"]
        d["tflops"] = d["flops"] / (d["total_ms"] * 1e-3) / 1e12 if d["total_ms"] > 0 else 0.0
    return out
