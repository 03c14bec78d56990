"""Per-launch GPU timing of the library's kernels with HIP events.

``record()`` is a context manager: while it is active every GEMM, attention,
LayerNorm, cross-entropy and embedding launch made through :mod:`resihp.ops` is
bracketed by two ``torch.cuda.Event``s on the stream it is enqueued on (the
current stream), labelled with the kernel instantiation it selects and annotated
with its algorithmic FLOPs (MFMA kernels) or algorithmic bytes (bandwidth
kernels: every input read once, every output written once).  After a
``torch.cuda.synchronize()``, ``summary()`` gives per-label launch counts, mean
duration, achieved TFLOP/s and GB/s.  Inactive, it costs one attribute check per
call.
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
def launch(label: str, flops: float = 0.0, nbytes: float = 0.0):
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
        _active.append((label, flops, nbytes, start, end))


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
    """{label: {"launches", "mean_ms", "total_ms", "flops_per_launch", "tflops", "bytes_per_launch", "gbps"}}."""
    out: dict = {}
    for label, flops, nbytes, s, e in events:
        ms = s.elapsed_time(e)
        d = out.setdefault(label, {"launches": 0, "total_ms": 0.0, "flops": 0.0, "bytes": 0.0})
        d["launches"] += 1
        d["total_ms"] += ms
        d["flops"] += flops
        d["bytes"] += nbytes
    for d in out.values():
        d["mean_ms"] = d["total_ms"] / d["launches"]
        d["flops_per_launch"] = d["flops"] / d["launches"]
        d["bytes_per_launch"] = d["bytes"] / d["launches"]
        d["tflops"] = d["flops"] / (d["total_ms"] * 1e-3) / 1e12 if d["total_ms"] > 0 else 0.0
        d["gbps"] = d["bytes"] / (d["total_ms"] * 1e-3) / 1e9 if d["total_ms"] > 0 else 0.0
    return out


# ---------------------------------------------------------------------------
# rocprofv3 database summaries (python -m resihp.profiling ...)
# ---------------------------------------------------------------------------
def library_sources_digest() -> str:
    """sha256 over the library's kernel sources (csrc/*), its C header and its build script (which
    holds the compiler flags): the identity of the kernels a counter summary describes."""
    import hashlib
    from pathlib import Path

    pkg_root = Path(__file__).resolve().parents[1]
    files = sorted((pkg_root / "csrc").glob("*")) + [pkg_root.parent / "include" / "resihp_hip.h",
                                                     pkg_root / "build.py"]
    h = hashlib.sha256()
    for f in files:
        if f.is_file():
            h.update(f.name.encode())
            h.update(f.read_bytes())
    return h.hexdigest()

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


def counters_markdown(fetch_db: str, write_db: str, mfma_db: str | None, copy_mib: int, dominant: str) -> str:
    """Per-kernel HBM read / write MB per launch and MFMA busy of three --pmc runs (FETCH_SIZE;
    WRITE_SIZE; SQ_VALU_MFMA_BUSY_CYCLES + GRBM_GUI_ACTIVE), each counter scaled by what it reads
    for `copy_kernel<16>` copying `copy_mib` MiB (a transfer of known size), plus the lines
    bench.py reads: the traffic of `dominant` and the sources digest of the measured library."""
    fetch = counter_table(fetch_db)
    write = counter_table(write_db)
    mfma = counter_table(mfma_db) if mfma_db else {}
    copy_kib = copy_mib * 1024.0
    f_scale = copy_kib / fetch["copy_kernel<16>"]["FETCH_SIZE"]
    w_scale = copy_kib / write["copy_kernel<16>"]["WRITE_SIZE"]
    out = [f"Calibration: `copy_kernel<16>` copies {copy_mib} MiB ({copy_kib:.0f} KiB read and written) per dispatch; "
           f"FETCH_SIZE reads {fetch['copy_kernel<16>']['FETCH_SIZE']:.0f} KiB and WRITE_SIZE "
           f"{write['copy_kernel<16>']['WRITE_SIZE']:.0f} KiB for it, so FETCH_SIZE is scaled by {f_scale:.3f} and "
           f"WRITE_SIZE by {w_scale:.3f}.  MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x GRBM_GUI_ACTIVE / 8 XCDs).",
           "", "| kernel | HBM read MB/launch | HBM write MB/launch | MFMA busy |", "|---|---:|---:|---:|"]
    for k in sorted(set(fetch) | set(write)):
        if k == "copy_kernel<16>":
            continue
        r = fetch.get(k, {}).get("FETCH_SIZE", 0.0) * f_scale * 1024 / 1e6
        w = write.get(k, {}).get("WRITE_SIZE", 0.0) * w_scale * 1024 / 1e6
        m = mfma.get(k, {})
        busy = ""
        if m.get("GRBM_GUI_ACTIVE"):
            busy = f"{100.0 * m.get('SQ_VALU_MFMA_BUSY_CYCLES', 0.0) / (1024 * m['GRBM_GUI_ACTIVE'] / 8):.1f}%"
        out.append(f"| `{k}` | {r:.1f} | {w:.1f} | {busy} |")
    t = (fetch[dominant]["FETCH_SIZE"] * f_scale + write[dominant]["WRITE_SIZE"] * w_scale) * 1024
    out += ["", f"traffic_bytes_per_launch {dominant} = {t:.0f}", "", f"library_sources_sha256 = {library_sources_digest()}"]
    return "\n".join(out)


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
    m = sub.add_parser("counters-md", help="markdown HBM / MFMA summary of FETCH_SIZE, WRITE_SIZE, MFMA runs")
    m.add_argument("--fetch", required=True)
    m.add_argument("--write", required=True)
    m.add_argument("--mfma")
    m.add_argument("--copy-mib", type=int, required=True)
    m.add_argument("--dominant", required=True)
    args = ap.parse_args(argv)
    if args.cmd == "kernels":
        print(kernel_table(args.db, args.steps))
    elif args.cmd == "counters":
        print(json.dumps(counter_table(args.db), indent=1, sort_keys=True))
    else:
        print(counters_markdown(args.fetch, args.write, args.mfma, args.copy_mib, args.dominant))
    return 0


if __name__ == "__main__":
    raise SystemExit(_main())
