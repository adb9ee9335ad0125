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


def _agent_shape(agent_csv: Optional[str]) -> Tuple[int, int]:
    """(XCDs, SIMDs) of the GPU agent in a rocprofv3 ``*_agent_info.csv``; MI355X's
    (8, 1024) when no file is given."""
    import csv
    import os

    if agent_csv and os.path.isfile(agent_csv):
        with open(agent_csv, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Agent_Type") == "GPU":
                    return int(row["Num_Xcc"]), int(row["Simd_Count"])
    return 8, 1024


def summarize_mfma(csv_path: str, agent_csv: Optional[str] = None, top: int = 12, clock_ghz: float = 2.4) -> str:
    """Per-kernel MFMA and LDS figures from a rocprofv3 ``--pmc`` run, as a Markdown
    table.  Counters are summed over the device for each dispatch and averaged over
    dispatches.  GRBM_GUI_ACTIVE counts active cycles on every XCD, so a dispatch
    lasts GRBM_GUI_ACTIVE / XCDs cycles; the MFMA pipe's busy share is
    SQ_VALU_MFMA_BUSY_CYCLES / (those cycles x SIMDs); fp32 MFMA flops are
    SQ_INSTS_VALU_MFMA_MOPS_F32 x 512, their rate uses ``clock_ghz``.  LDS bank
    conflicts are given as a share of SQ_LDS_IDX_ACTIVE cycles.  Columns whose
    counters the run did not collect are left empty."""
    import csv
    import os
    from collections import OrderedDict

    if not os.path.isfile(csv_path):
        raise FileNotFoundError(f"no rocprofv3 counter file at {csv_path}")
    xcds, simds = _agent_shape(agent_csv)
    per: "OrderedDict[str, Dict[str, float]]" = OrderedDict()
    kname: Dict[str, str] = {}
    with open(csv_path, newline="") as f:
        for row in csv.DictReader(f):
            d = row["Dispatch_Id"]
            per.setdefault(d, defaultdict(float))[row["Counter_Name"]] += float(row["Counter_Value"])
            kname[d] = row["Kernel_Name"]
    by_kernel: Dict[str, List[Dict[str, float]]] = defaultdict(list)
    for d, ctrs in per.items():
        by_kernel[kname[d]].append(ctrs)

    def avg(lst, key):
        vals = [c[key] for c in lst if key in c]
        return sum(vals) / len(vals) if vals else None

    rows = []
    for name, lst in by_kernel.items():
        gui = avg(lst, "GRBM_GUI_ACTIVE")
        cyc = gui / xcds if gui else None
        busy = avg(lst, "SQ_VALU_MFMA_BUSY_CYCLES")
        mops = avg(lst, "SQ_INSTS_VALU_MFMA_MOPS_F32")
        mfma = avg(lst, "SQ_INSTS_VALU_MFMA_F32") or avg(lst, "SQ_INSTS_MFMA")
        valu = avg(lst, "SQ_INSTS_VALU")
        lds_i = avg(lst, "SQ_INSTS_LDS")
        bank = avg(lst, "SQ_LDS_BANK_CONFLICT")
        lds_act = avg(lst, "SQ_LDS_IDX_ACTIVE")
        rows.append((cyc or 0.0, name, len(lst), cyc,
                     None if not (busy and cyc) else 100.0 * busy / (cyc * simds),
                     None if not (mops and cyc) else mops * 512.0 / (cyc / (clock_ghz * 1e9)) / 1e12,
                     None if not (valu and mfma) else (valu - mfma) / mfma,
                     None if not (lds_i and mfma) else lds_i / mfma,
                     None if not (bank and lds_act) else 100.0 * bank / lds_act))
    rows.sort(key=lambda r: -r[0] * r[2])

    def f(v, fmt):
        return "" if v is None else format(v, fmt)

    out = ["| kernel | dispatches | cycles per dispatch | MFMA busy | fp32 MFMA TFLOP/s | non-MFMA VALU per MFMA "
           "| LDS instructions per MFMA | LDS bank-conflict share of LDS-active cycles |",
           "|---|---:|---:|---:|---:|---:|---:|---:|"]
    for _w, name, n, cyc, busy, tf, valu_r, lds_r, bank_r in rows[:top]:
        out.append(f"| `{name[:110]}` | {n} | {f(cyc, '.0f')} | {f(busy, '.1f')}{'%' if busy is not None else ''} | "
                   f"{f(tf, '.1f')} | {f(valu_r, '.2f')} | {f(lds_r, '.2f')} | "
                   f"{f(bank_r, '.1f')}{'%' if bank_r is not None else ''} |")
    return "\n".join(out)


if __name__ == "__main__":
    import sys

    if len(sys.argv) == 3 and sys.argv[1] == "--pmc":
        print(summarize_pmc(sys.argv[2]))
    elif len(sys.argv) in (3, 4) and sys.argv[1] == "--mfma":
        print(summarize_mfma(sys.argv[2], sys.argv[3] if len(sys.argv) == 4 else None))
    elif len(sys.argv) == 2 and not sys.argv[1].startswith("-"):
        print(summarize_rocpd(sys.argv[1]))
    else:
        raise SystemExit("usage: python -m boundflow_amd.profiling <rocprofv3 *_results.db>\n"
                         "       python -m boundflow_amd.profiling --pmc <rocprofv3 *_counter_collection.csv>\n"
                         "       python -m boundflow_amd.profiling --mfma <*_counter_collection.csv> [<*_agent_info.csv>]")
