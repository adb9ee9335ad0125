"""Optional per-launch timing of the library's kernels with HIP events.

When a ``LaunchTimer`` is active, each launch of the named kernel families is
bracketed by ``torch.cuda.Event`` records on the stream the kernel is launched
on (the caller's current stream), taken right around the library call, with
the algorithmic flop and byte counts of that launch.  Nothing is synchronized
until ``summary()`` is called.
"""

from __future__ import annotations

from collections import defaultdict
from contextlib import contextmanager
from typing import Dict, List, Optional, Tuple

import torch

_active: Optional["LaunchTimer"] = None


class LaunchTimer:
    """``spin_cycles`` > 0 queues a bounded spin kernel (``torch.cuda._sleep``)
    ahead of each timed launch.  A launch-bound sequence issued from Python
    leaves the device idle between launches, and a start event recorded on an
    idle stream completes before its kernel is even submitted; the spin holds
    the device while the host records the start event and submits the kernel,
    so the two events bracket the kernel's execution.  Only for timing runs
    whose wall time is not measured."""

    def __init__(self, spin_cycles: int = 0) -> None:
        self.records: List[Tuple[str, float, float, torch.cuda.Event, torch.cuda.Event]] = []
        self.spin_cycles = int(spin_cycles)

    def summary(self) -> Dict[str, Dict[str, float]]:
        torch.cuda.synchronize()
        agg: Dict[str, Dict[str, float]] = defaultdict(lambda: {"launches": 0, "ms": 0.0, "flops": 0.0, "bytes": 0.0})
        for name, flops, nbytes, s, e in self.records:
            a = agg[name]
            a["launches"] += 1
            a["ms"] += s.elapsed_time(e)
            a["flops"] += flops
            a["bytes"] += nbytes
        out = {}
        for name, a in agg.items():
            sec = a["ms"] / 1e3
            out[name] = dict(a)
            out[name]["avg_ms"] = a["ms"] / max(1, a["launches"])
            out[name]["tflops"] = a["flops"] / sec / 1e12 if sec > 0 else 0.0
            out[name]["gbps"] = a["bytes"] / sec / 1e9 if sec > 0 else 0.0
        return out


@contextmanager
def timing(timer: LaunchTimer):
    global _active
    prev = _active
    _active = timer
    try:
        yield timer
    finally:
        _active = prev


_pending: Optional[list] = None   # [name, flops, bytes, start event, end event] of the bracketed launch


@contextmanager
def launch(name: str, flops: float, nbytes: float):
    """Time the first library call inside the block (no-op unless a
    LaunchTimer is active).  The events are recorded by the call itself,
    immediately around the foreign function, so host work that prepares the
    arguments -- during which a launch-bound device idles -- is not counted."""
    global _pending
    t = _active
    if t is None:
        yield
        return
    _pending = [name, float(flops), float(nbytes), None, None]
    try:
        yield
    finally:
        rec, _pending = _pending, None
        if rec is not None and rec[3] is not None and rec[4] is not None:
            t.records.append(tuple(rec))


def begin_call() -> None:
    if _pending is not None and _pending[3] is None:
        if _active is not None and _active.spin_cycles > 0:
            torch.cuda._sleep(_active.spin_cycles)
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        _pending[3] = ev


def end_call() -> None:
    if _pending is not None and _pending[3] is not None and _pending[4] is None:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        _pending[4] = ev


def spin_cycles(ms: float) -> int:
    """Cycle count of a ``torch.cuda._sleep`` spin of about ``ms`` milliseconds on
    the current device (calibrated with events)."""
    probe = 1 << 20
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    torch.cuda._sleep(probe)
    e.record()
    e.synchronize()
    return max(1, int(probe / max(s.elapsed_time(e), 1e-3) * ms))


def summarize_rocpd(db_path: str, top: int = 12) -> str:
    """Per-kernel dispatch count / average / total duration from a rocprofv3
    ``*_results.db`` (kernel-trace run), as a Markdown table."""
    import sqlite3

    import os

    if not os.path.isfile(db_path):
        raise FileNotFoundError(f"no rocprofv3 database at {db_path}")
    con = sqlite3.connect(f"file:{db_path}?mode=ro", uri=True)
    q = ("select s.kernel_name, count(*), avg(d.end - d.start), sum(d.end - d.start) "
         "from rocpd_kernel_dispatch d join rocpd_info_kernel_symbol s on d.kernel_id = s.id "
         "group by s.kernel_name order by 4 desc")
    rows = list(con.execute(q))
    total = sum(r[3] for r in rows) or 1
    out = ["| kernel | calls | avg (us) | total (ms) | share |", "|---|---:|---:|---:|---:|"]
    for name, n, avg, tot in rows[:top]:
        out.append(f"| `{name.removesuffix('.kd')}` | {n} | {avg / 1e3:.2f} | {tot / 1e6:.3f} | "
                   f"{100.0 * tot / total:.1f}% |")
    return "\n".join(out)


def summarize_pmc(csv_path: str, top: int = 12) -> str:
    """Per-kernel dispatch count and average counter value per dispatch from a
    rocprofv3 ``--pmc ... --output-format csv`` run (``*_counter_collection.csv``),
    as a Markdown table; counters summed over the device for each dispatch."""
    import csv
    import os
    from collections import OrderedDict

    if not os.path.isfile(csv_path):
        raise FileNotFoundError(f"no rocprofv3 counter file at {csv_path}")
    per_dispatch: "OrderedDict[tuple, float]" = OrderedDict()
    names = {}
    with open(csv_path, newline="") as f:
        for row in csv.DictReader(f):
            key = (row["Dispatch_Id"], row["Counter_Name"])
            per_dispatch[key] = per_dispatch.get(key, 0.0) + float(row["Counter_Value"])
            names[row["Dispatch_Id"]] = (row["Kernel_Name"], row.get("Grid_Size", ""))
    agg: Dict[Tuple[str, str], List[float]] = defaultdict(list)
    for (disp, ctr), v in per_dispatch.items():
        agg[(names[disp][0], ctr)].append(v)
    rows = sorted(agg.items(), key=lambda kv: -sum(kv[1]))
    out = ["| kernel | counter | dispatches | average per dispatch | total |", "|---|---|---:|---:|---:|"]
    for (name, ctr), vals in rows[:top]:
        out.append(f"| `{name[:100]}` | {ctr} | {len(vals)} | {sum(vals) / len(vals):.1f} | {sum(vals):.1f} |")
    return "\n".join(out)


if __name__ == "__main__":
    import sys

    if len(sys.argv) == 3 and sys.argv[1] == "--pmc":
        print(summarize_pmc(sys.argv[2]))
    elif len(sys.argv) == 2 and not sys.argv[1].startswith("-"):
        print(summarize_rocpd(sys.argv[1]))
    else:
        raise SystemExit("usage: python -m boundflow_amd.profiling <rocprofv3 *_results.db>\n"
                         "       python -m boundflow_amd.profiling --pmc <rocprofv3 *_counter_collection.csv>")
