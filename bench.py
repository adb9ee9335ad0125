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

    python bench.py [--steps K] [--warmup W] [--config C2|C1|C3|C4|C5] [--cpu-seconds S]
    python bench.py --calibrate-copy MIB   # one plain device copy of MIB MiB, the
                                           # reference kernel for HBM byte counters
"""

from __future__ import annotations

import argparse
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
    ("C2", "crown_relu_linear_relu_fwd"): (1.0120e9, "profiles/hbm_traffic_dominant_kernels.md"),
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


def build_case(name: str):
    import torch
    from boundflow_amd import crown as hc
    from boundflow_amd import workloads as wl

    dev = torch.device("cuda:0")
    w = wl.make(name)
    wd = wl.to_device(w, dev)
    if name == "C2":
        def step():
            return hc.run_crown_all_intermediate(wd.module, wd.spec, linear_spec_C=wd.C)[0]
        units, unit = w.batch * w.num_specs, "bounds/s"
        desc = "C2: CROWN, all intermediate bounds by CROWN, MLP 784-500x6-10, B=256, Linf 0.015, 9 margin specs"
    elif name in ("C1", "C3"):
        def step():
            return hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
        units, unit = w.batch * w.num_specs, "bounds/s"
        desc = {"C1": "C1: IBP+CROWN, MLP 784-256-256-10, B=64, box eps 2/255 clamped, 9 margin specs",
                "C3": "C3: CROWN, CNN 3x32x32 conv16-conv32-fc100-fc10, B=128, Linf 2/255, 9 margin specs"}[name]
    elif name == "C4":
        from boundflow_amd import alpha_beta as hab

        def step():
            return hab.run_alpha_crown_from_crown_init(wd.module, wd.spec, linear_spec_C=wd.C, steps=20, lr=0.1)[0]
        units, unit = w.batch * w.num_specs, "bounds/s"
        desc = "C4: alpha-CROWN, CNN of C3, B=32, Linf 8/255, 20 Adam steps lr 0.1, alpha from CROWN"
    elif name == "C5":
        from boundflow_amd import bab as hbab

        def step():
            return hbab.evaluate_domain_batch(wd.module, wd.spec, linear_spec_C=wd.C,
                                              relu_split_state=wd.extra["splits"], steps=10, lr=0.2)
        units, unit = w.batch, "domains/s"
        desc = "C5: beta-CROWN BaB batch, MLP 784-256x4-10, 4096 domains, Linf 0.03, 1-12 splits, 10 steps"
    else:
        raise SystemExit(f"unknown config {name}")
    return w, step, units, unit, desc


def cpu_baseline(name: str, w, seconds: float):
    """Time the CPU oracle (PyTorch CPU restatement of the reference path) on a
    bounded sample of the same workload; returns throughput in the metric unit."""
    import torch
    from boundflow_amd import workloads as wl
    from oracle import alpha_beta_ref as ab
    from oracle import crown_ref as cr

    threads = torch.get_num_threads()
    done_units = 0
    elapsed = 0.0
    rounds = 0
    sample_b = {"C1": 16, "C2": 4, "C3": 16, "C4": 2, "C5": 64}[name]
    while elapsed < seconds and rounds < 64:
        sub = wl.subset(w, sample_b)
        t0 = time.perf_counter()
        if name == "C2":
            with torch.inference_mode():
                cr.run_crown_all_intermediate(sub.module, sub.spec, linear_spec_C=sub.C)
            done_units += sub.batch * sub.num_specs
        elif name in ("C1", "C3"):
            with torch.inference_mode():
                cr.run_crown_ibp(sub.module, sub.spec, linear_spec_C=sub.C)
            done_units += sub.batch * sub.num_specs
        elif name == "C4":
            _e, pre = cr.forward_ibp_trace(sub.module, sub.spec)
            init = ab.adaptive_alpha_init(pre)
            ab.run_alpha_beta_crown(sub.module, sub.spec, linear_spec_C=sub.C, steps=20, lr=0.1,
                                    warm_start_alpha=init, per_batch_params=True)
            done_units += sub.batch * sub.num_specs
        else:
            ab.evaluate_domain_batch(sub.module, sub.spec, linear_spec_C=sub.C,
                                     relu_split_state=sub.extra["splits"], steps=10, lr=0.2)
            done_units += sub.batch
        elapsed += time.perf_counter() - t0
        rounds += 1
    return {
        "value": done_units / elapsed,
        "cores": threads,
        "kind": "port",
        "sample": f"{rounds} x {sample_b}-input subsets of {name} ({done_units} units, {elapsed:.1f} s), "
                  f"PyTorch CPU fp32 restatement of the reference path, {threads} threads on {cpu_model()}",
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
    # Queries without host synchronization (C1, C3, C4) are launch-bound at these
    # batch sizes: they are captured once as a HIP graph and every timed step
    # replays the whole query (all kernels rerun on the same inputs; for C4 the
    # forward trace, the alpha initialisation and all 20 Adam steps).
    use_graph = args.config in ("C1", "C3", "C4") and not args.no_graph
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
        # per-kernel durations (the same in eager launches) for the roofline
        with profiling.timing(timer):
            for _ in range(args.steps):
                step()
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
                   "launch": "hip_graph replay" if use_graph else "eager"},
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
