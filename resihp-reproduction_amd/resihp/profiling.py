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


# ---------------------------------------------------------------------------
# rocprofv3 database summaries (python -m resihp.profiling ...)
# ---------------------------------------------------------------------------
def _short_name(name: str) -> str:
    """'void (anonymous namespace)::gemm_bf16_dma<...>((anonymous namespace)::GemmParams<...>)' or
    'void rh_gemm_impl::gemm_bf16_dma<...>(rh_gemm_impl::GemmParams<...>)' -> 'gemm_bf16_dma<...>':
    the return type, namespace qualifiers of the kernel and the parameter list are dropped."""
    n = name.replace("(anonymous namespace)::", "")
    if n.startswith("void "):
        n = n[5:]
    depth = 0
    for i, ch in enumerate(n):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            n = n[:i]
            break
    # namespace qualifiers before the template arguments: keep what follows the last '::' there
    head = n.split("<", 1)[0]
    if "::" in head:
        n = n[len(head.rsplit("::", 1)[0]) + 2:]
    return n


def kernel_table(db_path: str, steps: int) -> str:
    """Markdown table of a --kernel-trace --stats database: calls, mean and per-step time."""
    import sqlite3

    con = sqlite3.connect(db_path)
    rows = con.execute("select name, total_calls, total_duration, average from top_kernels").fetchall()
    out = ["| kernel | calls | mean us | us per step | % |", "|---|---:|---:|---:|---:|"]
    total = sum(r[2] for r in rows)
    for name, calls, dur, avg in rows:
        out.append(f"| `{_short_name(name)}` | {calls} | {avg:.1f} | {dur / steps:.1f} | {100 * dur / total:.1f} |")
    out.append(f"| **all kernels** | | | **{total / steps:.1f}** | |")
    return "\n".join(out)


def counter_table(db_path: str) -> dict:
    """{kernel: {counter: mean per dispatch}} of a --pmc database (counters summed over the
    hardware instances of each dispatch)."""
    import sqlite3

    con = sqlite3.connect(db_path)
    q = ("select dispatch_id, kernel_name, counter_name, sum(value) from counters_collection "
         "group by dispatch_id, counter_name")
    acc: dict = {}
    for _, kname, cname, value in con.execute(q):
        d = acc.setdefault(_short_name(kname), {}).setdefault(cname, [])
        d.append(value)
    return {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in acc.items()}


def _main(argv=None) -> int:
    import argparse
    import json

    ap = argparse.ArgumentParser(prog="python -m resihp.profiling")
    sub = ap.add_subparsers(dest="cmd", required=True)
    k = sub.add_parser("kernels", help="markdown kernel table of a --kernel-trace --stats run")
    k.add_argument("db")
    k.add_argument("--steps", type=int, default=1, help="steps the trace covers (for per-step times)")
    c = sub.add_parser("counters", help="per-kernel mean counter values of a --pmc run (JSON)")
    c.add_argument("db")
    args = ap.parse_args(argv)
    if args.cmd == "kernels":
        print(kernel_table(args.db, args.steps))
    else:
        print(json.dumps(counter_table(args.db), indent=1, sort_keys=True))
    return 0


if __name__ == "__main__":
    raise SystemExit(_main())
