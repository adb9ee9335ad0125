#!/usr/bin/env python3
"""Throughput of the HIP bound-propagation hot path on one MI355X.

Default workload ("C2"): CROWN with every
intermediate pre-activation bound computed by CROWN on the fp32 MLP
784-500x6-10, batch 256, Linf eps 0.015, 9 margin specs per input.  One step
is one full query over the batch: IBP forward trace, five layer-by-layer CROWN
refinements (C = I, M = 256 x 500 coefficient rows) and the final spec bound.
The metric is final (lower, upper) bound pairs per second (2304 per step).

Prints ONE JSON line with the throughput, the roofline position of the
dominant kernel (timed with HIP events on the launch stream inside the timed
region) and a CPU baseline (the PyTorch CPU restatement of the reference path
timed on a bounded sample on this host).

    python bench.py [--steps K] [--warmup W] [--config C2|C1|C3|C4|C5|D1] [--cpu-seconds S]

D1 (not a BASELINE configuration) measures the DAG path: CROWN on a residual MLP.
    python bench.py --calibrate-copy MIB   # one plain device copy of MIB MiB, the
                                           # reference kernel for HBM byte counters
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import platform
import sys
import time

PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 matrix peak
PEAK_HBM_GBPS = 8000.0          # MI355X HBM3E

# HBM bytes per launch of a dominant kernel, measured with rocprofv3 --pmc
# FETCH_SIZE and WRITE_SIZE over one query (each scaled by what the counter
# reads for a 1 GiB device copy: x2.0 and x1.0), averaged over the launch mix
# of that query.  Keyed by (config, kernel family); other pairs report null.
MEASURED_TRAFFIC = {
    ("C2", "crown_relu_linear_relu_fwd"): (1.1600e9, "profiles/hbm_traffic_dominant_kernels.md"),
    ("C5", "crown_relu_linear_relu_fwd"): (1.3720e8, "profiles/hbm_traffic_dominant_kernels.md"),
    ("C5", "grad_gemm"): (1.0079e8, "profiles/hbm_traffic_dominant_kernels.md"),
}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def hip_runner(name: str):
    """The HIP path of a configuration as a function of a device workload."""
    from boundflow_amd import crown as hc

    if name == "C2":
        return lambda wd: hc.run_crown_all_intermediate(wd.module, wd.spec, linear_spec_C=wd.C)[0]
    if name in ("C1", "C3", "D1"):
        return lambda wd: hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
    if name == "C4":
        from boundflow_amd import alpha_beta as hab
        return lambda wd: hab.run_alpha_crown_from_crown_init(wd.module, wd.spec, linear_spec_C=wd.C, steps=20,
                                                              lr=0.1)[0]
    if name == "C5":
        from boundflow_amd import bab as hbab
        return lambda wd: hbab.evaluate_domain_batch(wd.module, wd.spec, linear_spec_C=wd.C,
                                                     relu_split_state=wd.extra["splits"], steps=10, lr=0.2)
    raise SystemExit(f"unknown config {name}")


def build_case(name: str):
    import torch
    from boundflow_amd import workloads as wl

    dev = torch.device("cuda:0")
    w = wl.make(name)
    wd = wl.to_device(w, dev)
    run = hip_runner(name)

    def step():
        return run(wd)

    if name == "C5":
        units, unit = w.batch, "domains/s"
    else:
        units, unit = w.batch * w.num_specs, "bounds/s"
    desc = {"C1": "C1: IBP+CROWN, MLP 784-256-256-10, B=64, box eps 2/255 clamped, 9 margin specs",
            "C2": "C2: CROWN, all intermediate bounds by CROWN, MLP 784-500x6-10, B=256, Linf 0.015, 9 margin specs",
            "C3": "C3: CROWN, CNN 3x32x32 conv16-conv32-fc100-fc10, B=128, Linf 2/255, 9 margin specs",
            "C4": "C4: alpha-CROWN, CNN of C3, B=32, Linf 8/255, 20 Adam steps lr 0.1, alpha from CROWN",
            "C5": "C5: beta-CROWN BaB batch, MLP 784-256x4-10, 4096 domains, Linf 0.03, 1-12 splits, 10 steps",
            "D1": "D1: CROWN on a residual MLP (DAG), 784-256 stem, 4 blocks 256-512-256 with identity skips, "
                  "head 10, B=256, Linf 0.002, 9 margin specs"}[name]
    return w, step, units, unit, desc


def intermediate_bounds(w) -> int:
    """Pre-activation bounds refined by CROWN per C2 step: every ReLU input after the first, per input."""
    from boundflow_amd import crown as hc

    shapes = hc.parse_chain(w.module, w.spec).relu_shapes
    widths = [int(torch_numel(s)) for s in shapes.values()]
    return w.batch * sum(widths[1:])


def torch_numel(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


def _oracle_run(name: str, sub):
    """The oracle's result for a workload (the computation the CPU baseline times)."""
    import torch
    from oracle import alpha_beta_ref as ab
    from oracle import crown_ref as cr

    if name == "C2":
        with torch.inference_mode():
            return cr.run_crown_all_intermediate(sub.module, sub.spec, linear_spec_C=sub.C)
    if name in ("C1", "C3", "D1"):
        with torch.inference_mode():
            return cr.run_crown_ibp(sub.module, sub.spec, linear_spec_C=sub.C)
    if name == "C4":
        _e, pre = cr.forward_ibp_trace(sub.module, sub.spec)
        init = ab.adaptive_alpha_init(pre)
        return ab.run_alpha_beta_crown(sub.module, sub.spec, linear_spec_C=sub.C, steps=20, lr=0.1,
                                       warm_start_alpha=init, per_batch_params=True)
    return ab.evaluate_domain_batch(sub.module, sub.spec, linear_spec_C=sub.C,
                                    relu_split_state=sub.extra["splits"], steps=10, lr=0.2)


def _bounds(name: str, res):
    if name == "C5":
        return res["lower"], res["upper"]
    r = res[0] if isinstance(res, tuple) else res
    return r.lower, r.upper


def parity_summary(name: str, sub, ref) -> dict:
    """HIP result on the CPU-baseline sample against the oracle's result on it.
    The contract: rtol 1e-5 / atol 1e-6 on both bounds (C1-C3); rtol 1e-4 /
    atol 1e-4 on the optimised lower bound (C4, C5: Adam trajectories amplify fp32
    rounding).  Rows outside it count as explained when the fp64 oracle run is
    as far from the fp32 oracle as the HIP value is.  Also: verdict mismatches,
    near ties (|min_s lb| < 1e-4) and, for the BaB batch, statuses and branching."""
    import torch
    from boundflow_amd import workloads as wl
    from oracle import parity

    got = hip_runner(name)(wl.to_device(sub, torch.device("cuda:0")))
    torch.cuda.synchronize()
    g_lo, g_hi = (t.cpu() for t in _bounds(name, got))
    r_lo, r_hi = _bounds(name, ref)
    optimised = name in ("C4", "C5")
    rtol, atol = (1e-4, 1e-4) if optimised else (1e-5, 1e-6)
    keep = torch.isfinite(r_lo).all(dim=1)
    pick = (lambda lo, hi: lo[keep]) if optimised else (lambda lo, hi: torch.cat([lo[keep], hi[keep]]))
    rep = parity.compare(pick(g_lo, g_hi), pick(r_lo, r_hi), None, rtol=rtol, atol=atol)
    if rep.strict_violations:
        ref64 = _oracle_run(name, parity.to_float64(sub))
        e_lo, e_hi = _bounds(name, ref64)
        rep = parity.compare(pick(g_lo, g_hi), pick(r_lo, r_hi), pick(e_lo, e_hi), rtol=rtol, atol=atol)
    g_min = g_lo[keep].min(dim=1).values
    r_min = r_lo[keep].min(dim=1).values
    out = {"contract": f"rtol {rtol:g} atol {atol:g} on " + ("the optimised lower bound" if optimised else "both bounds"),
           "values": rep.n, "max_abs_err": rep.max_abs, "max_rel_err": rep.max_rel,
           "outside_contract": rep.strict_violations, "explained_by_fp64": rep.explained_by_fp32,
           "unexplained": rep.unexplained, "verdict_mismatches": int(((g_min >= 0) != (r_min >= 0)).sum()),
           "near_ties": int((r_min.abs() < 1e-4).sum())}
    if name == "C5":
        out["status_mismatches"] = int(((got["status"].cpu() == 1) != ref["certified"]).sum())
        names = got["relu_names"]
        layer, neuron = got["branch_layer"].cpu().tolist(), got["branch_neuron"].cpu().tolist()
        hip_branch = [None if l < 0 else (names[l], n) for l, n in zip(layer, neuron)]
        out["branch_mismatches"] = sum(bool(ref["feasible"][i]) and hip_branch[i] != ref["branch"][i]
                                       for i in range(len(hip_branch)))
    return out


def cpu_baseline(name: str, w, seconds: float):
    """Time the CPU oracle (PyTorch CPU restatement of the reference path) on a
    bounded sample of the same workload; returns throughput in the metric unit."""
    import torch
    from boundflow_amd import workloads as wl

    threads = torch.get_num_threads()
    done_units = 0
    elapsed = 0.0
    rounds = 0
    sample_b = {"C1": 16, "C2": 4, "C3": 16, "C4": 2, "C5": 64, "D1": 16}[name]
    first = None
    while elapsed < seconds and rounds < 4096:
        sub = wl.subset(w, sample_b)
        t0 = time.perf_counter()
        res = _oracle_run(name, sub)
        done_units += sub.batch if name == "C5" else sub.batch * sub.num_specs
        elapsed += time.perf_counter() - t0
        rounds += 1
        if first is None:
            first = (sub, res)
    return {
        "value": done_units / elapsed,
        "cores": threads,
        "kind": "port",
        "sample": f"{rounds} x {sample_b}-input subsets of {name} ({done_units} units, {elapsed:.1f} s), "
                  f"PyTorch CPU fp32 restatement of the reference path, {threads} threads on {cpu_model()}",
        "parity": parity_summary(name, *first),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="C2")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB")
    ap.add_argument("--no-graph", action="store_true", help="issue every launch from Python (no HIP graph replay)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only; the path shards by domain with no "
                                   "collective during bound computation, run with --gpus 1"}))
        return 2

    import torch
    from boundflow_amd import profiling

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device"}))
        return 1
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": 4 * n, "copy_bytes_written": 4 * n, "launches": 3}), flush=True)
        return 0
    w, step, units, unit, desc = build_case(args.config)
    # Queries without host synchronization (C1, C3, C4, C5) are captured once as a
    # HIP graph and every timed step replays the whole query (all kernels rerun on
    # the same inputs; for C4 the forward trace, the alpha initialisation and all
    # 20 Adam steps; for C5 the batch's forward trace, 10 alpha-beta steps and the
    # certification).  C1, C3 and C4 are launch-bound at these batch sizes; C5
    # leaves the device idle between launches for about 7 % of an eager batch.
    use_graph = args.config in ("C1", "C3", "C4", "C5", "D1") and not args.no_graph
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    timer = profiling.LaunchTimer()
    if use_graph:
        from boundflow_amd import graphs
        replay = graphs.CapturedQuery(step)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            replay()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        # Per-kernel durations (the same in eager launches) for the roofline, in a
        # separate pass after one untimed eager query (the first eager query after
        # the graph replays runs slow), with the garbage collector off: each timed
        # launch is preceded by a 0.2 ms spin so that its events bracket execution,
        # not the host's launch latency.
        step()
        timer = profiling.LaunchTimer(spin_cycles=profiling.spin_cycles(0.2))
        # a garbage-collection pause between a start event and its launch would outlast the spin
        gc.disable()
        try:
            with profiling.timing(timer):
                for _ in range(args.steps):
                    step()
            torch.cuda.synchronize()
        finally:
            gc.enable()
    else:
        with profiling.timing(timer):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                step()
            torch.cuda.synchronize()
            t1 = time.perf_counter()
    sec = t1 - t0
    kernels = timer.summary()
    dom_name, dom = max(kernels.items(), key=lambda kv: kv[1]["ms"]) if kernels else (None, None)
    roofline = None
    if dom is not None:
        traffic, source = MEASURED_TRAFFIC.get((args.config, dom_name), (None, None))
        common = {"kernel": dom_name, "traffic": traffic, "traffic_source": source,
                  "algorithmic_bytes_per_launch": round(dom["bytes"] / max(1, dom["launches"])),
                  "avg_launch_ms": round(dom["avg_ms"], 4), "launches": int(dom["launches"]),
                  "share_of_step": round(dom["ms"] / 1e3 / sec, 4),
                  "timing": "eager launches" if use_graph else "timed steps"}
        if dom["flops"] > 0:
            roofline = {"bound": "mfma", "achieved": round(dom["tflops"], 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(dom["tflops"] / PEAK_FP32_MFMA_TFLOPS, 4), **common}
        else:
            roofline = {"bound": "hbm", "achieved": round(dom["gbps"], 1), "peak": PEAK_HBM_GBPS,
                        "unit": "GB/s", "frac": round(dom["gbps"] / PEAK_HBM_GBPS, 4), **common}
    line = {
        "metric": "CROWN bounds/sec & BaB domains/sec on 1 GPU; % of HBM / fp32-MFMA roofline",
        "value": round(units * args.steps / sec, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Kaiming weights, uniform inputs)",
        "config": {"workload": desc, "units_per_step": units, "parallelism": "single GPU",
                   "launch": "hip_graph replay" if use_graph else "eager",
                   **({"intermediate_bounds_per_step": intermediate_bounds(w)} if args.config == "C2" else {})},
        "roofline": roofline,
        "kernels": {k: {"launches": int(v["launches"]), "avg_ms": round(v["avg_ms"], 4),
                        "tflops": round(v["tflops"], 3), "gbps": round(v["gbps"], 1)} for k, v in kernels.items()},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.config, w, args.cpu_seconds)
        line["cpu_baseline"]["unit"] = unit
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
