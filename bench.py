#!/usr/bin/env python3
"""Throughput of the HIP bound-propagation hot path on one MI355X.

Default workload ("C2"): CROWN with every
intermediate pre-activation bound computed by CROWN on the fp32 MLP
784-500x6-10, batch 256, Linf eps 0.015, 9 margin specs per input.  One step
is one full query over the batch: IBP forward trace, five layer-by-layer CROWN
refinements (C = I, M = 256 x 500 coefficient rows) and the final spec bound.
The metric is final (lower, upper) bound pairs per second (2304 per step).

Prints ONE JSON line with the throughput, the roofline position of the
dominant kernel (timed with HIP events on the launch stream) and a CPU baseline
(the PyTorch CPU restatement of the reference path timed on the whole batch on
this host, with the parity of the HIP result against it).  With the default C2
workload the line also carries ``secondary``: the metric's other half, BaB
domains/s on the C5 domain batch (4096 subdomains of
the MLP 784-256x4-10, 10 alpha-beta steps each), and the bounds/s of the other
BASELINE configurations C1, C3 and C4, each with its own roofline, CPU
baseline and parity over its whole batch.

    python bench.py [--steps K] [--warmup W] [--config C2|C1|C3|C4|C5|D1] [--cpu-seconds S]

D1 (not a BASELINE configuration) measures the DAG path: CROWN on a residual MLP.
    python bench.py --calibrate-copy MIB   # one plain device copy of MIB MiB, the
                                           # reference kernel for HBM byte counters
    python bench.py --hbm-ceiling MIB      # attainable rates: fill, copy, read-only sum and a
                                           # write-bound product on MIB MiB buffers, and the
                                           # library's fp32 GEMM on the C2 / C5 contraction shapes
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
    ("C2", "crown_relu_linear_relu_fwd"): (1.2301e9, "profiles/hbm_traffic_dominant_kernels.md"),
    ("C5", "crown_relu_linear_relu_fwd"): (1.3250e8, "profiles/hbm_traffic_dominant_kernels.md"),
    ("C5", "grad_gemm"): (1.0040e8, "profiles/hbm_traffic_dominant_kernels.md"),
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


def executor_regions(name: str, dev):
    """The fused ReLU -> affine regions of the C1 (X1) or C3 (X3) network as the
    drop-in executor receives them (FusedReluAffineRequest, fused_crown.py:97-123):
    for every Linear / Conv2d layer whose output feeds a ReLU, the coefficient of
    the batch's 9 margin specs at that ReLU, the layer's weights, and synthetic
    relaxations (upper slope in [0.1, 1] with intercept in [0, 0.5], lower slope
    0 or 1, lower intercept 0)."""
    import torch
    from boundflow_amd import fused_crown as fc
    from boundflow_amd import workloads as wl

    w = wl.make("C1" if name == "X1" else "C3")
    ops = w.module.get_entry_task().ops
    params = w.module.params
    g = torch.Generator().manual_seed(17)
    B, S = w.batch, w.num_specs
    x = w.spec.center
    reqs = []
    for i, op in enumerate(ops):
        x_in = x
        if op.op_type == "linear":
            x = torch.nn.functional.linear(x, params[op.inputs[1]], params[op.inputs[2]])
        elif op.op_type == "conv2d":
            x = torch.nn.functional.conv2d(x, params[op.inputs[1]], params[op.inputs[2]], stride=op.attrs["stride"],
                                           padding=op.attrs["padding"])
        elif op.op_type == "relu":
            x = torch.relu(x)
        elif op.op_type == "flatten":
            x = x.flatten(1)
        feeds_relu = i + 1 < len(ops) and ops[i + 1].op_type == "relu" and ops[i + 1].inputs[0] == op.outputs[0]
        if op.op_type not in ("linear", "conv2d") or not feeds_relu:
            continue
        n = int(x[0].numel())
        au = torch.rand(B, n, generator=g) * 0.9 + 0.1
        bu = torch.rand(B, n, generator=g) * 0.5
        al = (torch.rand(B, n, generator=g) > 0.5).float()
        reqs.append(fc.FusedReluAffineRequest(
            kind=op.op_type, A_u=torch.randn(B, S, n, generator=g).to(dev), A_l=torch.randn(B, S, n, generator=g).to(dev),
            alpha_u=au.to(dev), alpha_l=al.to(dev), beta_u=bu.to(dev), beta_l=torch.zeros(B, n, device=dev),
            weight=params[op.inputs[1]].to(dev), bias=params[op.inputs[2]].to(dev),
            input_shape=tuple(int(d) for d in x_in.shape[1:]), output_shape=tuple(int(d) for d in x.shape[1:]),
            attrs=dict(op.attrs) if op.op_type == "conv2d" else {}))
    return w, reqs


def build_case(name: str):
    import torch
    from boundflow_amd import workloads as wl

    dev = torch.device("cuda:0")
    if name in ("X1", "X3"):
        from boundflow_amd import fused_crown as fc
        w, reqs = executor_regions(name, dev)
        ex = fc.HipFusedCrownExecutor()
        ctx = fc.FusedCrownExecutionContext()
        assert all(ex.supports(r, ctx) for r in reqs)

        def step():
            return [ex.run(r) for r in reqs]

        rows = sum(int(r.A_u.shape[0] * r.A_u.shape[1]) for r in reqs)
        desc = (f"{name}: HipFusedCrownExecutor.run on every ReLU -> affine region of the "
                f"{'C1 MLP' if name == 'X1' else 'C3 CNN'} ({len(reqs)} regions, B={w.batch}, 9 margin specs, "
                "upper and lower coefficients, synthetic relaxations)")
        return w, step, rows, "region rows/s", desc
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
    """The oracle's result for a workload: the computation the CPU baseline times.
    C5 times the reference's node-batch call (one per_batch_params alpha-beta
    evaluation of every domain, bab.py:1323)."""
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
    return ab.run_alpha_beta_crown(sub.module, sub.spec, linear_spec_C=sub.C, relu_split_state=sub.extra["splits"],
                                   steps=10, lr=0.2, per_batch_params=True)


def _bounds(name: str, res):
    if isinstance(res, dict):
        return res["lower"], res["upper"]
    r = res[0] if isinstance(res, tuple) else res
    return r.lower, r.upper


def parity_summary(name: str, w, ref) -> dict:
    """HIP result on the whole workload against the oracle's result on it, at the
    contract rtol 1e-5 / atol 1e-6 on both bounds: a value outside it counts as
    explained when the fp64 oracle is as far from the fp32 oracle as the HIP
    value is.  C4, C5 (optimised bounds): ``optimised_parity``.  Also: verdict
    mismatches and near ties (|min_s lb| < 1e-4)."""
    import torch
    from boundflow_amd import workloads as wl
    from oracle import parity

    if name in ("C4", "C5"):
        return optimised_parity(name, w)
    got = hip_runner(name)(wl.to_device(w, torch.device("cuda:0")))
    torch.cuda.synchronize()
    g_lo, g_hi = (t.cpu() for t in _bounds(name, got))
    r_lo, r_hi = _bounds(name, ref)
    pick = lambda lo, hi: torch.cat([lo, hi])   # noqa: E731
    strict = parity.compare(pick(g_lo, g_hi), pick(r_lo, r_hi), None)
    rep = strict
    if strict.strict_violations:
        e_lo, e_hi = _bounds(name, _oracle_run(name, parity.to_float64(w)))
        rep = parity.compare(pick(g_lo, g_hi), pick(r_lo, r_hi), pick(e_lo, e_hi))
    g_min = g_lo.min(dim=1).values
    r_min = r_lo.min(dim=1).values
    return {"contract": "rtol 1e-05 atol 1e-06 on both bounds", "values": rep.n, "max_abs_err": rep.max_abs,
            "max_rel_err": rep.max_rel, "outside_contract": rep.strict_violations,
            "explained_by_fp64": rep.explained_by_fp32, "unexplained": rep.unexplained,
            "verdict_mismatches": int(((g_min >= 0) != (r_min >= 0)).sum()),
            "near_ties": int((r_min.abs() < 1e-4).sum()), "sample": f"the whole batch ({w.batch} inputs)"}


def optimised_parity(name: str, w) -> dict:
    """C4 / C5: the HIP optimisation and the oracle's, both recorded step by step,
    over the whole batch.  ``outside_contract`` counts the final bounds outside
    rtol 1e-5 / atol 1e-6 (C4: both bounds; C5: the lower bound of the feasible
    domains); ``outside_band_1e-3`` the same at 1e-3.  Every domain outside the
    contract is traced (oracle/trajectory.py: the HIP trajectory checked step by
    step against the oracle at the HIP states, and the step at which the two
    trajectories part shown to be reachable by Adam within the gradients' fp32
    uncertainty); ``unexplained`` is 0 when the trace holds.  C5 also: certified
    counts, status and branching mismatches over the feasible domains, and the
    infeasible domains on each side."""
    import torch
    from boundflow_amd import alpha_beta as hab
    from boundflow_amd import bab as hbab
    from boundflow_amd import workloads as wl
    from oracle import alpha_beta_ref as ab
    from oracle import crown_ref as cr
    from oracle import parity
    from oracle import trajectory as tt

    wd = wl.to_device(w, torch.device("cuda:0"))
    hrec, srec = [], []
    if name == "C4":
        got, best_alpha, _b, _st = hab.run_alpha_crown_from_crown_init(wd.module, wd.spec, linear_spec_C=wd.C,
                                                                       steps=20, lr=0.1, record=hrec)
        torch.cuda.synchronize()
        _e, pre = cr.forward_ibp_trace(w.module, w.spec)
        ref = ab.run_alpha_beta_crown(w.module, w.spec, linear_spec_C=w.C, steps=20, lr=0.1,
                                      warm_start_alpha=ab.adaptive_alpha_init(pre), per_batch_params=True,
                                      record=srec)[0]
        wf, g_lo, g_hi, r_lo, r_hi, lr = w, got.lower.cpu(), got.upper.cpu(), ref.lower, ref.upper, 0.1
        best = {n: v.cpu() for n, v in best_alpha.items()}
        sample = range(w.batch)
        out = {}
    else:
        got = hbab.evaluate_domain_batch(wd.module, wd.spec, linear_spec_C=wd.C, relu_split_state=wd.extra["splits"],
                                         steps=10, lr=0.2, record=hrec)
        torch.cuda.synchronize()
        ref = ab.evaluate_domain_batch(w.module, w.spec, linear_spec_C=w.C, relu_split_state=w.extra["splits"],
                                       steps=10, lr=0.2, record=srec)
        status = got["status"].cpu()
        feas = ref["feasible"]
        idx = feas.nonzero().flatten()
        hrec = tt.slice_record(hrec, idx)
        wf = tt.sub_workload(w, idx)
        g_lo, g_hi, r_lo, r_hi, lr = got["lower"].cpu()[idx], got["upper"].cpu()[idx], ref["lower"][idx], None, 0.2
        best = {n: v.cpu()[idx] for n, v in got["alpha"].items()}
        sample = range(0, len(idx), 64)
        hip_cert = status == 1
        names = got["relu_names"]
        layer, neuron = got["branch_layer"].cpu().tolist(), got["branch_neuron"].cpu().tolist()
        hip_branch = [None if l < 0 else (names[l], n) for l, n in zip(layer, neuron)]
        out = {"certified": {"hip": int(hip_cert.sum()), "reference": int(ref["certified"].sum()), "of": w.batch},
               "infeasible": {"hip": int((status == 2).sum()), "reference": int((~feas).sum())},
               "status_mismatches": int((hip_cert != ref["certified"]).sum()) + int(((status == 2) != ~feas).sum()),
               "branch_mismatches": sum(hip_branch[i] != ref["branch"][i] for i in idx.tolist())}
    both_g = g_lo if r_hi is None else torch.cat([g_lo, g_hi])
    both_r = r_lo if r_hi is None else torch.cat([r_lo, r_hi])
    strict = parity.compare(both_g, both_r, None)
    band = parity.compare(both_g, both_r, None, rtol=1e-3, atol=1e-3)
    logs = []
    try:
        trace = tt.trace_run(wf, hrec, srec, g_lo, r_lo, lr, what=name, sample=sample, got_upper=g_hi,
                             ref_upper=r_hi, best_alpha=best, fp64_lower=lambda rows: _oracle_run(
                                 name, parity.to_float64(tt.sub_workload(wf, rows)))[0].lower, log=logs.append)
        unexplained, failure = 0, None
    except AssertionError as exc:
        trace, unexplained, failure = None, strict.strict_violations, str(exc)[:300]
    g_min, r_min = g_lo.min(dim=1).values, r_lo.min(dim=1).values
    res = {"contract": "rtol 1e-05 atol 1e-06 on the optimised " + ("lower bound of the feasible domains"
                                                                     if name == "C5" else "bounds"),
           "values": strict.n, "max_abs_err": strict.max_abs, "max_rel_err": strict.max_rel,
           "outside_contract": strict.strict_violations, "outside_band_1e-3": band.strict_violations,
           "traced_to_trajectory_divergence": strict.strict_violations if trace is not None else 0,
           "unexplained": unexplained, "trajectory_trace": trace,
           "verdict_mismatches": int(((g_min >= 0) != (r_min >= 0)).sum()),
           "near_ties": int((r_min.abs() < 1e-4).sum()),
           "sample": f"all {w.batch} domains" if name == "C5" else f"the whole batch ({w.batch} inputs)"}
    if failure is not None:
        res["trace_failure"] = failure
    res.update(out)
    return res


def cpu_baseline(name: str, w, seconds: float):
    """Time the CPU oracle (PyTorch CPU restatement of the reference path) on the
    whole workload, repeated while less than ``seconds`` have elapsed; returns the
    throughput in the metric unit and the parity of the HIP result against the
    first run."""
    import torch

    threads = torch.get_num_threads()
    done_units = 0
    elapsed = 0.0
    rounds = 0
    first = None
    while rounds == 0 or elapsed < seconds:
        t0 = time.perf_counter()
        res = _oracle_run(name, w)
        elapsed += time.perf_counter() - t0
        done_units += w.batch if name == "C5" else w.batch * w.num_specs
        rounds += 1
        if first is None:
            first = res
    what = "node-batch alpha-beta evaluations" if name == "C5" else "queries"
    return {
        "value": done_units / elapsed,
        "cores": threads,
        "kind": "port",
        "sample": f"{rounds} full-batch {what} of {name} ({done_units} units, {elapsed:.1f} s), PyTorch CPU fp32 "
                  f"restatement of the reference path, {threads} threads on {cpu_model()}",
        "parity": parity_summary(name, w, first),
    }


def _settle(run, warmup: int, seconds: float = 0.2) -> None:
    """Untimed runs right before the timed ones: at least ``warmup`` of them and at least
    ``seconds`` of sustained work.  A timed region of a few milliseconds (C1 and C3 take
    well under 0.3 ms per step) started on a device that has just been idle can catch its
    clocks still ramping up, which multiplies the measured step time by up to ten."""
    import torch
    t0 = time.perf_counter()
    n = 0
    while n < max(1, warmup) or time.perf_counter() - t0 < seconds:
        run()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def hbm_ceiling(mib: int, reps: int) -> dict:
    """Attainable HBM rates of plain streams over ``mib`` MiB buffers, each launch
    timed with HIP events on the current stream and averaged over ``reps``:
    fill (write only), copy (read + write, the runtime's blit), sum (read only) and
    a broadcast product out[d, r, k] = w[r, k] * s[d, k] whose small operands stay
    in L2 (the write-bound shape of the strided relaxation pass: 500 x 500 rows per
    domain, two outputs); and the vendor library's fp32 product (torch.mm, TF32 off)
    on the shapes of the C2 and C5 contractions."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.rand(n, device="cuda:0")
    dst = torch.empty_like(src)
    R = K = 500
    D = max(1, n // (2 * R * K))
    wm = torch.rand(R, K, device="cuda:0")
    s = torch.rand(D, 1, K, device="cuda:0")
    out_u = torch.empty(D, R, K, device="cuda:0")
    out_l = torch.empty(D, R, K, device="cuda:0")

    def bcast():
        torch.mul(wm, s, out=out_u)
        torch.mul(wm, s, out=out_l)

    cases = {
        "fill": (lambda: dst.fill_(1.0), 4 * n),
        "copy": (lambda: dst.copy_(src), 8 * n),
        "sum": (lambda: src.sum(), 4 * n),
        "broadcast_product_two_outputs": (bcast, 2 * 4 * D * R * K),
    }
    res = {"mib": mib, "reps": reps}
    # the vendor library's plain fp32 products on the shapes of the dominant contractions
    # (C2: 128000 x 500 rows against a 500 x 500 weight; C5: 36864 x 256 against 256 x 256),
    # full fp32: no TF32, no reduced precision
    torch.backends.cuda.matmul.allow_tf32 = False
    for M, N, K in ((128000, 500, 500), (36864, 256, 256)):
        a_m = torch.rand(M, K, device="cuda:0")
        w_m = torch.rand(N, K, device="cuda:0")
        c_m = torch.empty(M, N, device="cuda:0")
        mm = lambda: torch.mm(a_m, w_m.t(), out=c_m)   # noqa: E731
        _settle(mm, 3, seconds=0.3)
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(reps):
            mm()
        s1.record()
        s1.synchronize()
        ms = s0.elapsed_time(s1) / reps
        flops = 2.0 * M * N * K
        res[f"library_sgemm_{M}x{N}x{K}"] = {"flops": flops, "avg_ms": round(ms, 4),
                                             "tflops": round(flops / ms / 1e9, 2),
                                             "frac_of_fp32_mfma_peak": round(flops / ms / 1e9 / PEAK_FP32_MFMA_TFLOPS, 4)}
        # this library's plain contraction (bf_gemm, store epilogue) on the same operands
        from boundflow_amd import _lib
        st = _lib.stream_handle()
        ours = lambda: _lib.call("bf_gemm", _lib.ptr(a_m), K, _lib.ptr(w_m), K, 1, 0, _lib.ptr(c_m), N,  # noqa: E731
                                 M, N, K, st)
        _settle(ours, 3, seconds=0.3)
        s0.record()
        for _ in range(reps):
            ours()
        s1.record()
        s1.synchronize()
        ms = s0.elapsed_time(s1) / reps
        res[f"bf_gemm_{M}x{N}x{K}"] = {"flops": flops, "avg_ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 2),
                                       "frac_of_fp32_mfma_peak": round(flops / ms / 1e9 / PEAK_FP32_MFMA_TFLOPS, 4)}
        del a_m, w_m, c_m
    for name, (fn, nbytes) in cases.items():
        _settle(fn, 3, seconds=0.3)
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(reps):
            fn()
        s1.record()
        s1.synchronize()
        ms = s0.elapsed_time(s1) / reps
        res[name] = {"bytes": nbytes, "avg_ms": round(ms, 4), "gbps": round(nbytes / ms / 1e6, 1),
                     "frac_of_peak": round(nbytes / ms / 1e6 / PEAK_HBM_GBPS, 4)}
    return res


def measure(name: str, steps: int, warmup: int, no_graph: bool):
    """One configuration: throughput of ``steps`` timed steps after ``warmup``, the
    per-kernel durations of the library's launches and the dominant kernel's
    roofline position.  Returns (record, workload, unit)."""
    import torch
    from boundflow_amd import profiling

    w, step, units, unit, desc = build_case(name)
    # Every configuration's query is free of host synchronization, so one query is
    # captured as a HIP graph and every timed step replays it (all kernels rerun on
    # the same inputs; C2: the IBP trace, five CROWN refinements of 128 000 rows and
    # the final bound; C4: the forward trace, the alpha initialisation and 20 Adam
    # steps; C5: the batch's forward trace, 10 alpha-beta steps and the
    # certification).  Python issue of the eager launches leaves the device idle
    # between them (C2: about 6 % of a step).
    use_graph = not no_graph
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    timer = profiling.LaunchTimer()
    if use_graph:
        from boundflow_amd import graphs
        replay = graphs.CapturedQuery(step)
        torch.cuda.synchronize()
        _settle(replay, warmup)
        t0 = time.perf_counter()
        for _ in range(steps):
            replay()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        del replay
        # Per-kernel durations (the same in eager launches) for the roofline, in a
        # separate pass after one untimed eager query (the first eager query after
        # the graph replays runs slow), with the garbage collector off: each timed
        # launch is preceded by a 0.2 ms spin so that its events bracket execution,
        # not the host's launch latency.
        step()
        timer = profiling.LaunchTimer(spin_cycles=profiling.spin_cycles(0.2))
        gc.disable()
        try:
            with profiling.timing(timer):
                for _ in range(steps):
                    step()
            torch.cuda.synchronize()
        finally:
            gc.enable()
    else:
        _settle(step, warmup)
        with profiling.timing(timer):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
            t1 = time.perf_counter()
    sec = t1 - t0
    kernels = timer.summary()
    dom_name, dom = max(kernels.items(), key=lambda kv: kv[1]["ms"]) if kernels else (None, None)
    roofline = None
    if dom is not None:
        traffic, source = MEASURED_TRAFFIC.get((name, dom_name), (None, None))
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
    config = {"workload": desc, "units_per_step": units, "parallelism": "single GPU",
              "launch": "hip_graph replay" if use_graph else "eager"}
    if name == "C2":
        config["intermediate_bounds_per_step"] = intermediate_bounds(w)
    record = {"value": round(units * steps / sec, 2), "unit": unit, "steps": steps,
              "ms_per_step": round(sec / steps * 1e3, 4), "config": config, "roofline": roofline,
              "kernels": {k: {"launches": int(v["launches"]), "avg_ms": round(v["avg_ms"], 4),
                              "tflops": round(v["tflops"], 3), "gbps": round(v["gbps"], 1)}
                          for k, v in kernels.items()}}
    return record, w, unit


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="C2")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--secondary-cpu-seconds", type=float, default=8.0,
                    help="CPU baseline time of each secondary configuration")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB")
    ap.add_argument("--hbm-ceiling", type=int, default=0, metavar="MIB",
                    help="time plain fill / copy / read streams of MIB MiB (the attainable HBM ceiling)")
    ap.add_argument("--no-graph", action="store_true", help="issue every launch from Python (no HIP graph replay)")
    ap.add_argument("--no-secondary", action="store_true",
                    help="C2 alone, without the C5 domains/s and C1 / C3 / C4 bounds/s records")
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
    if args.hbm_ceiling:
        print(json.dumps(hbm_ceiling(args.hbm_ceiling, max(args.steps, 5))), flush=True)
        return 0
    head, w, unit = measure(args.config, args.steps, args.warmup, args.no_graph)
    line = {
        "metric": "CROWN bounds/sec & BaB domains/sec on 1 GPU; % of HBM / fp32-MFMA roofline",
        "value": head["value"],
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Kaiming weights, uniform inputs)",
        "config": head["config"],
        "roofline": head["roofline"],
        "kernels": head["kernels"],
    }
    if not args.no_cpu and not args.config.startswith("X"):   # X1 / X3: executor profile entries, no CPU leg
        line["cpu_baseline"] = cpu_baseline(args.config, w, args.cpu_seconds)
        line["cpu_baseline"]["unit"] = unit
    # the metric's second half (BaB domains/s on the C5 domain batch) and the other BASELINE
    # configurations' bounds/s (C1, C3, C4), each measured in the same run with its own
    # roofline, CPU baseline and whole-batch parity
    if args.config == "C2" and not args.no_secondary:
        del w
        line["secondary"] = []
        for name, metric in (("C5", "BaB domains/sec (beta-CROWN domain batch)"),
                             ("C1", "CROWN bounds/sec (IBP + CROWN, MLP)"), ("C3", "CROWN bounds/sec (CNN)"),
                             ("C4", "CROWN bounds/sec (alpha-CROWN, CNN)")):
            gc.collect()
            torch.cuda.empty_cache()
            sec_rec, ws, unit_s = measure(name, args.steps, args.warmup, args.no_graph)
            sec_rec = {"metric": metric, "config_id": name, **sec_rec}
            if not args.no_cpu:
                sec_rec["cpu_baseline"] = cpu_baseline(name, ws, args.secondary_cpu_seconds)
                sec_rec["cpu_baseline"]["unit"] = unit_s
            line["secondary"].append(sec_rec)
            del ws
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
