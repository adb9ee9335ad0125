"""Write golden input/output vectors from the reference implementation.

Runs ONLY in the build container, where the reference checkout is mounted
read-only (default ``/root/reference``, override with ``BOUNDFLOW_REFERENCE``).
It imports the reference's own Python (boundflow.runtime.*), feeds it the
seeded workloads of ``boundflow_amd.workloads`` and stores the outputs as small
``.npz`` fixtures next to this script.  Inputs are regenerated from the seed
by the tests; each fixture keeps a checksum of the inputs it was made from so a
generator change is detected.

Usage:  python tests/golden/make_golden.py [tag-substring ...]
"""

from __future__ import annotations

import hashlib
import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))
REF = os.environ.get("BOUNDFLOW_REFERENCE", "/root/reference")
sys.path.insert(0, REF)

from boundflow.domains.interval import IntervalState as RIntervalState  # noqa: E402
from boundflow.ir.task import BFTaskModule as RModule  # noqa: E402
from boundflow.ir.task import BoundTask as RTask  # noqa: E402
from boundflow.ir.task import TaskKind as RKind  # noqa: E402
from boundflow.ir.task import TaskOp as ROp  # noqa: E402
from boundflow.ir.task import BufferSpec as RBufferSpec  # noqa: E402
from boundflow.ir.task import StoragePlan as RStoragePlan  # noqa: E402
from boundflow.ir.task_graph import TaskBufferDep as RDep  # noqa: E402
from boundflow.ir.task_graph import TaskDepEdge as REdge  # noqa: E402
from boundflow.ir.task_graph import TaskGraph as RGraph  # noqa: E402
from boundflow.runtime.scheduler import run_ibp_scheduled as r_run_ibp_scheduled  # noqa: E402
from boundflow.runtime.task_executor import PythonTaskExecutor as RPythonTaskExecutor  # noqa: E402
from boundflow.runtime import alpha_beta_crown as rabc  # noqa: E402
from boundflow.runtime import alpha_crown as rac  # noqa: E402
from boundflow.runtime import crown_ibp as rci  # noqa: E402
from boundflow.runtime import fused_crown as rfc  # noqa: E402
from boundflow.runtime.perturbation import BoxPerturbation as RBox  # noqa: E402
from boundflow.runtime.task_executor import InputSpec as RSpec  # noqa: E402

from boundflow_amd import workloads as wl  # noqa: E402
from boundflow_amd.spec import BoxPerturbation  # noqa: E402


def to_ref_module(m):
    t = m.get_entry_task()
    ops = [ROp(op_type=o.op_type, name=o.name, inputs=list(o.inputs), outputs=list(o.outputs), attrs=dict(o.attrs))
           for o in t.ops]
    task = RTask(task_id=t.task_id, kind=RKind.INTERVAL_IBP, ops=ops, input_values=list(t.input_values),
                 output_values=list(t.output_values))
    return RModule(tasks=[task], entry_task_id=t.task_id, bindings={"params": dict(m.params)})


def to_ref_module_graph(m):
    """Every task, the storage plan and the task graph of a multi-task module."""
    def buf(b):
        return RBufferSpec(buffer_id=b.buffer_id, dtype=b.dtype, shape=list(b.shape))
    sp = m.storage_plan
    plan = RStoragePlan(buffers={k: buf(v) for k, v in sp.buffers.items()}, value_to_buffer=dict(sp.value_to_buffer),
                        physical_buffers={k: buf(v) for k, v in sp.physical_buffers.items()},
                        logical_to_physical=dict(sp.logical_to_physical))
    tasks = []
    for t in m.tasks:
        ops = [ROp(op_type=o.op_type, name=o.name, inputs=list(o.inputs), outputs=list(o.outputs),
                   attrs=dict(o.attrs)) for o in t.ops]
        tasks.append(RTask(task_id=t.task_id, kind=RKind.INTERVAL_IBP, ops=ops, input_values=list(t.input_values),
                           output_values=list(t.output_values), input_buffers=list(t.input_buffers),
                           output_buffers=list(t.output_buffers)))
    g = m.task_graph
    graph = RGraph(task_ids=list(g.task_ids), edges=[
        REdge(src_task_id=e.src_task_id, dst_task_id=e.dst_task_id,
              deps=[RDep(src_value=d.src_value, src_buffer_id=d.src_buffer_id, dst_value=d.dst_value,
                         dst_buffer_id=d.dst_buffer_id) for d in e.deps]) for e in g.edges])
    return RModule(tasks=tasks, entry_task_id=m.entry_task_id, bindings={"params": dict(m.params)},
                   storage_plan=plan, task_graph=graph)


def to_ref_spec(spec):
    p = spec.perturbation
    if isinstance(p, BoxPerturbation):
        return RSpec(value_name=spec.value_name, center=spec.center, perturbation=RBox(lower=p.lower, upper=p.upper))
    if str(getattr(p, "p", "inf")) not in ("inf", "Linf"):
        from boundflow.runtime.perturbation import LpBallPerturbation as RLp
        return RSpec(value_name=spec.value_name, center=spec.center, perturbation=RLp(p=int(p.p), eps=float(p.eps)))
    return RSpec.linf(value_name=spec.value_name, center=spec.center, eps=float(p.eps))


def checksum(*tensors) -> str:
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.detach().cpu().contiguous().numpy().tobytes())
    return h.hexdigest()


def workload_checksum(w) -> str:
    ts = [w.spec.center, w.C] + [w.module.params[k] for k in sorted(w.module.params)]
    if "splits" in w.extra:
        ts += [w.extra["splits"][k] for k in sorted(w.extra["splits"])]
    return checksum(*ts)


def save(name: str, **arrays):
    out = {}
    for k, v in arrays.items():
        if torch.is_tensor(v):
            v = v.detach().cpu().numpy()
        out[k] = np.asarray(v)
    np.savez_compressed(HERE / f"{name}.npz", **out)
    print("wrote", name, {k: getattr(v, "shape", None) for k, v in out.items()})


def golden_crown(w, tag, pre_rows=None):
    rm = to_ref_module(w.module)
    rs = to_ref_spec(w.spec)
    with torch.inference_mode():
        b = rci.run_crown_ibp_mlp(rm, rs, linear_spec_C=w.C)
        env, pre = rci._forward_ibp_trace_mlp(rm, rs)
    arrays = {"lower": b.lower, "upper": b.upper, "checksum": workload_checksum(w)}
    for i, (name, st) in enumerate(pre.items()):
        arrays[f"pre{i}_lower"] = st.lower[:pre_rows]
        arrays[f"pre{i}_upper"] = st.upper[:pre_rows]
    save(tag, **arrays)


def golden_all_intermediate(w, tag):
    """Layer-by-layer CROWN refinement composed from the reference functions
    (native_intermediate_refinement.py:923-988 pattern)."""
    rm = to_ref_module(w.module)
    rs = to_ref_spec(w.spec)
    with torch.inference_mode():
        env, pre = rci._forward_ibp_trace_mlp(rm, rs)
        names = list(pre.keys())
        for name in names[1:]:
            numel = int(pre[name].lower[0].numel())
            eye = torch.eye(numel)
            b = rci.run_crown_ibp_mlp_from_forward_trace(rm, rs, interval_env=env, relu_pre=pre,
                                                          linear_spec_C=eye, output_value=name)
            cur = pre[name]
            pre[name] = RIntervalState(lower=torch.maximum(cur.lower, b.lower), upper=torch.minimum(cur.upper, b.upper))
        final = rci.run_crown_ibp_mlp_from_forward_trace(rm, rs, interval_env=env, relu_pre=pre, linear_spec_C=w.C)
    arrays = {"lower": final.lower, "upper": final.upper, "checksum": workload_checksum(w)}
    for i, (name, st) in enumerate(pre.items()):
        arrays[f"pre{i}_lower"] = st.lower
        arrays[f"pre{i}_upper"] = st.upper
    save(tag, **arrays)


def golden_alpha_cnn(w, tag):
    rm = to_ref_module(w.module)
    rs = to_ref_spec(w.spec)
    env, pre = rci._forward_ibp_trace_mlp(rm, rs)
    # alpha "from CROWN": native_alpha_beta_optimizer_schedule.py:635-653
    from boundflow.runtime.native_alpha_beta_optimizer_schedule import _initial_alpha_state
    from boundflow.runtime.native_alpha_beta_optimization_state import NativeAlphaBetaOptimizerPolicy
    policy = NativeAlphaBetaOptimizerPolicy(steps=int(w.extra["steps"]), lr=float(w.extra["lr"]),
                                            alpha_initialization_mode="adaptive")
    init = _initial_alpha_state(pre, policy=policy)
    bounds, alpha, beta, stats = rabc.run_alpha_beta_crown_mlp(
        rm, rs, linear_spec_C=w.C, steps=int(w.extra["steps"]), lr=float(w.extra["lr"]),
        warm_start_alpha=rac.AlphaState(init), per_batch_params=True)
    arrays = {"lower": bounds.lower, "upper": bounds.upper, "checksum": workload_checksum(w)}
    for i, (name, a) in enumerate(alpha.alpha_by_relu_input.items()):
        arrays[f"alpha{i}"] = a
        arrays[f"init{i}"] = init[name]
    save(tag, **arrays)


def golden_bab_batch(w, tag):
    rm = to_ref_module(w.module)
    splits = w.extra["splits"]
    D = int(w.spec.center.shape[0])
    feasible = torch.zeros(D, dtype=torch.bool)
    for d in range(D):
        sub = RSpec.linf(value_name="input", center=w.spec.center[d:d + 1], eps=float(w.spec.perturbation.eps))
        try:
            rci._forward_ibp_trace_mlp(rm, sub, relu_split_state={k: v[d:d + 1] for k, v in splits.items()})
            feasible[d] = True
        except ValueError:
            feasible[d] = False
    idx = feasible.nonzero().flatten()
    sub = RSpec.linf(value_name="input", center=w.spec.center[idx], eps=float(w.spec.perturbation.eps))
    bounds, alpha, beta, stats = rabc.run_alpha_beta_crown_mlp(
        rm, sub, linear_spec_C=w.C[idx], relu_split_state={k: v[idx] for k, v in splits.items()},
        steps=int(w.extra["steps"]), lr=float(w.extra["lr"]), alpha_init=float(w.extra["alpha_init"]),
        beta_init=float(w.extra["beta_init"]), per_batch_params=True)
    names = list(splits.keys())
    layer = np.full(D, -1, dtype=np.int64)
    neuron = np.full(D, -1, dtype=np.int64)
    for j, d in enumerate(idx.tolist()):
        ch = stats.branch_choices[j]
        if ch is not None:
            layer[d] = names.index(ch[0])
            neuron[d] = ch[1]
    lower = torch.full((D, int(w.C.shape[1])), float("nan"))
    upper = torch.full((D, int(w.C.shape[1])), float("nan"))
    lower[idx] = bounds.lower.detach()
    upper[idx] = bounds.upper.detach()
    certified = torch.zeros(D, dtype=torch.bool)
    certified[idx] = lower[idx].min(dim=1).values >= -1e-6
    save(tag, lower=lower, upper=upper, feasible=feasible, certified=certified, branch_layer=layer,
         branch_neuron=neuron, checksum=workload_checksum(w))


def golden_fused_region(tag, kind):
    g = torch.Generator().manual_seed(7)
    D, S = 3, 4
    if kind == "linear":
        N, P = 12, 9
        out_shape, in_shape = (N,), (P,)
        weight = torch.randn(N, P, generator=g)
        attrs = {}
    else:
        out_shape, in_shape = (4, 4, 4), (3, 8, 8)
        N = 64
        weight = torch.randn(4, 3, 4, 4, generator=g)
        attrs = {"stride": (2, 2), "padding": (1, 1), "dilation": (1, 1), "groups": 1, "output_padding": (0, 0)}
    A_u = torch.randn(D, S, N, generator=g)
    A_l = torch.randn(D, S, N, generator=g)
    A_u[0, 0, :3] = torch.tensor([0.0, 1.0, -1.0])
    A_l[0, 0, :3] = torch.tensor([0.0, -1.0, 1.0])
    l = torch.randn(D, N, generator=g)
    u = l + torch.rand(D, N, generator=g) * 2
    au, bu, al, bl = rci._relu_relax(l, u)
    bias = torch.randn(weight.shape[0], generator=g)
    req = rfc.FusedReluAffineRequest(kind=kind, A_u=A_u, A_l=A_l, alpha_u=au, alpha_l=al, beta_u=bu, beta_l=bl,
                                     weight=weight, bias=bias, input_shape=in_shape, output_shape=out_shape,
                                     attrs=attrs)
    res = rfc.TorchDenseFusedCrownReference().run(req)
    save(tag, A_u=A_u, A_l=A_l, l=l, u=u, alpha_u=au, alpha_l=al, beta_u=bu, beta_l=bl, weight=weight, bias=bias,
         A_prev_u=res.A_prev_u, A_prev_l=res.A_prev_l, bias_delta_u=res.bias_delta_u, bias_delta_l=res.bias_delta_l)


def golden_task_ibp(w, tag):
    """PythonTaskExecutor.run_ibp (task_executor.py:127-358) on the entry task."""
    with torch.inference_mode():
        out = RPythonTaskExecutor().run_ibp(to_ref_module(w.module), to_ref_spec(w.spec))
    save(tag, lower=out.lower, upper=out.upper, checksum=workload_checksum(w))


def golden_task_ibp_scheduled(w, tag):
    """run_ibp_scheduled (scheduler.py:160-255) over the three-task split of the DAG program."""
    rm = to_ref_module_graph(wl.split_ibp_dag(w))
    with torch.inference_mode():
        out = r_run_ibp_scheduled(rm, to_ref_spec(w.spec))
    save(tag, lower=out.lower, upper=out.upper, checksum=workload_checksum(w))


from tests.golden_util import BAB_SOLVE_CASES  # noqa: E402


def count_certificates():
    """Wrap the reference's certificate to count the nodes it closes and the calls that
    evaluate at least one first-layer halfspace (for the fixtures' records)."""
    orig = rabc._is_infeasible_split_first_layer_convex_combo
    orig_collect = rabc._collect_first_layer_split_halfspaces
    box = {"calls": 0, "closed": 0, "halfspace_calls": 0}

    def wrapped(module, spec, *, relu_split_state, **kw):
        out = orig(module, spec, relu_split_state=relu_split_state, **kw)
        box["calls"] += 1
        box["closed"] += int(bool(out[0]))
        return out

    def collect(*a, **kw):
        hs = orig_collect(*a, **kw)
        box["halfspace_calls"] += int(len(hs) > 0)
        return hs

    rabc._is_infeasible_split_first_layer_convex_combo = wrapped
    rabc._collect_first_layer_split_halfspaces = collect

    def restore():
        rabc._is_infeasible_split_first_layer_convex_combo = orig
        rabc._collect_first_layer_split_halfspaces = orig_collect
    return box, restore


def golden_bab_solve(tag):
    """solve_bab_mlp (bab.py:631-1528) on the small BaB workload."""
    from boundflow.runtime.bab import BabConfig as RBabConfig
    from boundflow.runtime.bab import solve_bab_mlp as r_solve
    toy, kw = BAB_SOLVE_CASES[tag]
    w = wl.make_bab_case(**toy)
    counts, restore = count_certificates()
    try:
        res = r_solve(to_ref_module(w.module), to_ref_spec(w.spec), linear_spec_C=w.C, config=RBabConfig(**kw))
    finally:
        restore()
    print(tag, "certificate calls", counts)
    per = res.per_example
    status_code = {"proven": 0, "unsafe": 1, "unknown": 2}
    save(tag, status=status_code[res.status], nodes_visited=res.nodes_visited, nodes_evaluated=res.nodes_evaluated,
         nodes_expanded=res.nodes_expanded, max_queue=res.max_queue, batch_rounds=res.batch_rounds,
         avg_batch_fill_rate=res.avg_batch_fill_rate, best_lower=res.best_lower, best_upper=res.best_upper,
         per_status=np.array([status_code[r.status] for r in per]),
         per_visited=np.array([r.nodes_visited for r in per]),
         per_evaluated=np.array([r.nodes_evaluated for r in per]),
         per_expanded=np.array([r.nodes_expanded for r in per]),
         per_best_lower=np.array([r.best_lower for r in per]),
         per_best_upper=np.array([r.best_upper for r in per]),
         certificate_calls=counts["calls"], certificate_closed=counts["closed"],
         certificate_halfspace_calls=counts["halfspace_calls"], checksum=workload_checksum(w))


def golden_lp(tag):
    """Every reference path over an L2 (tag lp_reference_p2) or L1 (lp_reference_p1) ball,
    on the networks of tests/golden_util.lp_case: run_crown_ibp_mlp on an MLP and a CNN,
    alpha-CROWN from the CROWN slopes (10 steps), the first-layer certificate on the
    geometric known answers and on 48 C5 first-layer nodes (flags and max_value), and a
    whole solve_bab_mlp search."""
    from boundflow.runtime.bab import BabConfig as RBabConfig
    from boundflow.runtime.bab import solve_bab_mlp as r_solve
    from boundflow.runtime.perturbation import LpBallPerturbation as RLp
    from tests.golden_util import LP_BAB, lp_case, lp_cert_nodes
    from tests.test_oracle_certificate import LP_KATS, first_layer_module
    p = int(tag[-1])
    arrays = {}
    for kind in ("mlp", "cnn"):
        w = lp_case(kind, p)
        with torch.inference_mode():
            b = rci.run_crown_ibp_mlp(to_ref_module(w.module), to_ref_spec(w.spec), linear_spec_C=w.C)
        arrays[f"crown_{kind}_lower"], arrays[f"crown_{kind}_upper"] = b.lower, b.upper
        arrays[f"crown_{kind}_checksum"] = workload_checksum(w)
    # alpha-CROWN: adaptive init (native_alpha_beta_optimizer_schedule.py:635-653), 10 steps, lr 0.1
    w = lp_case("alpha", p)
    rm, rs = to_ref_module(w.module), to_ref_spec(w.spec)
    _env, pre = rci._forward_ibp_trace_mlp(rm, rs)
    from boundflow.runtime.native_alpha_beta_optimizer_schedule import _initial_alpha_state
    from boundflow.runtime.native_alpha_beta_optimization_state import NativeAlphaBetaOptimizerPolicy
    init = _initial_alpha_state(pre, policy=NativeAlphaBetaOptimizerPolicy(steps=10, lr=0.1,
                                                                          alpha_initialization_mode="adaptive"))
    bounds, _alpha, _beta, _stats = rabc.run_alpha_beta_crown_mlp(
        rm, rs, linear_spec_C=w.C, steps=10, lr=0.1, warm_start_alpha=rac.AlphaState(init), per_batch_params=True)
    arrays["alpha_lower"], arrays["alpha_upper"] = bounds.lower, bounds.upper
    arrays["alpha_checksum"] = workload_checksum(w)
    # the certificate: known answers and C5 first-layer nodes
    for name, (Wk, bk, sk, _expect) in LP_KATS.items():
        m = first_layer_module(torch.tensor(Wk), torch.tensor(bk))
        spec = RSpec(value_name="input", center=torch.zeros(1, 2), perturbation=RLp(p=p, eps=1.0))
        ok, _r, cert = rabc._is_infeasible_split_first_layer_convex_combo(
            to_ref_module(m), spec, relu_split_state={"h1": torch.tensor([sk], dtype=torch.int8)})
        arrays[f"kat_{name}_flag"] = int(bool(ok))
        arrays[f"kat_{name}_value"] = float(cert["max_value"]) if cert is not None else float("nan")
    w = lp_case("cert_c5", p)
    name, rows = lp_cert_nodes(w, p)
    rm = to_ref_module(w.module)
    flags, values = [], []
    for r in range(int(rows.shape[0])):
        spec = to_ref_spec(wl.subset(w, r + 1).spec)
        spec = RSpec(value_name=spec.value_name, center=spec.center[r:r + 1], perturbation=spec.perturbation)
        ok, _r, cert = rabc._is_infeasible_split_first_layer_convex_combo(rm, spec,
                                                                          relu_split_state={name: rows[r:r + 1]})
        flags.append(int(bool(ok)))
        values.append(float(cert["max_value"]) if cert is not None else float("nan"))
    arrays["cert_c5_flag"], arrays["cert_c5_value"] = np.array(flags), np.array(values)
    arrays["cert_c5_checksum"] = workload_checksum(w)
    # a whole search
    w = lp_case("bab", p)
    res = r_solve(to_ref_module(w.module), to_ref_spec(w.spec), linear_spec_C=w.C, config=RBabConfig(**LP_BAB[p][1]))
    per = res.per_example
    code = {"proven": 0, "unsafe": 1, "unknown": 2}
    arrays.update(bab_per_status=np.array([code[q.status] for q in per]),
                  bab_per_visited=np.array([q.nodes_visited for q in per]),
                  bab_per_evaluated=np.array([q.nodes_evaluated for q in per]),
                  bab_per_expanded=np.array([q.nodes_expanded for q in per]),
                  bab_per_best_lower=np.array([q.best_lower for q in per]),
                  bab_per_best_upper=np.array([q.best_upper for q in per]),
                  bab_max_queue=res.max_queue, bab_batch_rounds=res.batch_rounds, bab_checksum=workload_checksum(w))
    print(tag, "certificate C5 closed", sum(flags), "of", len(flags), "bab", [q.status for q in per])
    save(tag, **arrays)


def golden_cert_conv(tag):
    """The reference's first-layer certificate (_is_infeasible_split_first_layer_convex_combo,
    alpha_beta_crown.py:391-532) on C3's first conv layer (3x32x32 input, 16x16x16
    neurons), one node per call with one split neuron: a split against a stable neuron's
    sign is infeasible by itself ("single_halfspace_max_negative", with its max_value), one
    with the sign or on an ambiguous neuron is not.  24 nodes over the first 8 inputs."""
    w = wl.subset(wl.make_c3(), 8)
    rm = to_ref_module(w.module)
    with torch.inference_mode():
        _env, pre = rci._forward_ibp_trace_mlp(rm, to_ref_spec(w.spec))
    lo = pre["h0"].lower.reshape(8, -1)
    hi = pre["h0"].upper.reshape(8, -1)
    g = torch.Generator().manual_seed(41)
    rows = []
    for e in range(8):
        pos = (lo[e] > 0).nonzero().flatten()
        neg = (hi[e] < 0).nonzero().flatten()
        amb = ((lo[e] < 0) & (hi[e] > 0)).nonzero().flatten()
        pick = lambda t: int(t[int(torch.randint(0, int(t.numel()), (1,), generator=g))])  # noqa: E731
        rows.append((e, pick(pos), -1))                      # against the sign: infeasible
        rows.append((e, pick(neg), 1 if e % 2 == 0 else -1))   # +1 infeasible, -1 with the sign
        rows.append((e, pick(amb) if amb.numel() else pick(pos), 1 if e % 2 else -1))
    flags, values = [], []
    for e, n, sg in rows:
        split = torch.zeros(1, 16 * 16 * 16, dtype=torch.int8)
        split[0, n] = sg
        spec = RSpec.linf(value_name="input", center=w.spec.center[e:e + 1], eps=float(w.spec.perturbation.eps))
        ok, _reason, cert = rabc._is_infeasible_split_first_layer_convex_combo(
            rm, spec, relu_split_state={"h0": split.reshape(1, 16, 16, 16)})
        flags.append(int(bool(ok)))
        values.append(float(cert["max_value"]) if cert is not None else float("nan"))
    print(tag, "infeasible", sum(flags), "of", len(rows))
    save(tag, example=np.array([r[0] for r in rows]), neuron=np.array([r[1] for r in rows]),
         sign=np.array([r[2] for r in rows]), flag=np.array(flags), max_value=np.array(values),
         checksum=workload_checksum(w))


def golden_shared_alpha(tag):
    g = torch.Generator().manual_seed(5)
    m = wl.build_mlp([20, 16, 16, 5], gen=g, bias_std=0.1)
    x = torch.rand(6, 20, generator=g)
    labels = torch.randint(0, 5, (6,), generator=g)
    C = wl.margin_spec(labels, 5)
    from boundflow_amd.spec import InputSpec
    spec = InputSpec.linf(value_name="input", center=x, eps=0.1)
    w = wl.Workload("shared", m, spec, C, labels)
    rm = to_ref_module(m)
    bounds, state, _stats = rac.run_alpha_crown_mlp(rm, to_ref_spec(spec), linear_spec_C=C, steps=8, lr=0.2)
    arrays = {"lower": bounds.lower, "upper": bounds.upper, "checksum": workload_checksum(w)}
    for i, a in enumerate(state.alpha_by_relu_input.values()):
        arrays[f"alpha{i}"] = a
    save(tag, **arrays)


from tests.frontend_models import VNNLIB_SOURCES, frontend_nets, planned_module_json, vnnlib_c1_property  # noqa: E402,E501


def golden_frontend(tag):
    """import_torch (frontends/pytorch/frontend.py:21-80) + plan_interval_ibp_v0
    (planner/interval_v0.py:10-76) of the frontend nets: the planned modules' fields."""
    from boundflow.frontends.pytorch.frontend import import_torch as r_import_torch
    from boundflow.planner import plan_interval_ibp_v0 as r_plan
    arrays = {}
    for name, (net, x) in frontend_nets().items():
        tm = r_plan(r_import_torch(net, (x,), export_mode="export", normalize=True))
        arrays[name] = np.array(planned_module_json(tm))
    save(tag, **arrays)


def golden_vnnlib(tag):
    """parse_vnnlib_box_query (frontends/vnnlib.py) of the VNNLIB sources: the query IR as a dict and its hash."""
    import json
    from boundflow.frontends.vnnlib import parse_vnnlib_box_query as r_parse
    arrays = {}
    sources = dict(VNNLIB_SOURCES)
    sources["c1_property0"] = vnnlib_c1_property(0)
    for name, text in sources.items():
        q = r_parse(text, query_id=f"{name}:0")
        arrays[name] = np.array(json.dumps({"dict": q.to_dict(), "stable_hash": q.stable_hash()}, sort_keys=True))
    save(tag, **arrays)


from tests.frontend_models import native_bab_toy, native_toy  # noqa: E402
from tests.golden_util import (ALPHA_CROWN_OBJECTIVE_CASES, OBJECTIVE_CASES, c3_box, dag_case,  # noqa: E402
                               objective_workload)


def golden_objectives(tag):
    """run_alpha_beta_crown_mlp (runtime/alpha_beta_crown.py:643-941) with the
    objectives and spec reductions of OBJECTIVE_CASES on a small MLP with splits:
    the best bounds of each."""
    w, splits = objective_workload()
    names = list(splits)
    rm, rs = to_ref_module(w.module), to_ref_spec(w.spec)
    arrays = {"checksum": workload_checksum(w)}
    for case, kw in OBJECTIVE_CASES.items():
        try:
            b, _a, _bt, _st = rabc.run_alpha_beta_crown_mlp(rm, rs, linear_spec_C=w.C, relu_split_state=splits,
                                                            steps=8, lr=0.1, **kw)
        except ValueError:
            raise
        arrays[f"{case}_lower"] = b.lower
        arrays[f"{case}_upper"] = b.upper
    for n in names:
        arrays[f"split_{n}"] = splits[n]
    save(tag, **arrays)


def golden_alpha_crown_objectives(tag):
    """run_alpha_crown_mlp (runtime/alpha_crown.py:137-261) with the objectives of
    ALPHA_CROWN_OBJECTIVE_CASES on the objectives_mlp problem (shared alpha, the
    same splits): the best bounds and alpha of each."""
    from boundflow.runtime.alpha_crown import run_alpha_crown_mlp as r_alpha
    w, splits = objective_workload()
    rm, rs = to_ref_module(w.module), to_ref_spec(w.spec)
    arrays = {"checksum": workload_checksum(w)}
    for case, kw in ALPHA_CROWN_OBJECTIVE_CASES.items():
        b, st, _stats = r_alpha(rm, rs, linear_spec_C=w.C, relu_split_state=splits, steps=8, lr=0.1, **kw)
        arrays[f"{case}_lower"] = b.lower
        arrays[f"{case}_upper"] = b.upper
        for n, a in st.alpha_by_relu_input.items():
            arrays[f"{case}_alpha_{n}"] = a
    save(tag, **arrays)


# tag -> (problem, config fields)
NATIVE_CASES = {
    "native_toy_b4": ("toy", dict(max_nodes=15, max_depth=3, expansion_batch_size=2, max_eval_batch_size=4,
                                  threshold=1e6)),
    "native_toy_budget": ("toy", dict(max_nodes=7, max_depth=3, expansion_batch_size=2, max_eval_batch_size=4,
                                      threshold=1e6)),
    "native_mlp": ("mlp", dict(max_nodes=41, max_depth=6, expansion_batch_size=3, max_eval_batch_size=8,
                               threshold=0.0)),
}


def golden_native(tag):
    """run_native_relu_split_bab (runtime/native_relu_split_bab_runtime.py:592-789)."""
    import json
    from boundflow.runtime.native_relu_split_bab_runtime import NativeReluSplitBabConfig as RCfg
    from boundflow.runtime.native_relu_split_bab_runtime import run_native_relu_split_bab as r_run
    prob, cfg = NATIVE_CASES[tag]
    module, spec, C = native_toy() if prob == "toy" else native_bab_toy()
    trace = r_run(to_ref_module(module), to_ref_spec(spec), linear_spec_C=C, run_id=tag, config=RCfg(**cfg))

    def br(b):
        return None if b is None else [b.relu_input, b.neuron_index, b.lower, b.upper, b.width]

    out = {"status": trace.status, "termination_reason": trace.termination_reason,
           "frontier": list(trace.final_frontier_node_ids), "max_queue_size": trace.max_queue_size,
           "stacks": trace.native_stack_count,
           "evaluations": [{"node_id": e.node.node_id, "parent": e.node.parent_node_id, "depth": e.node.depth,
                            "lower": e.lower, "upper": e.upper, "priority": e.priority,
                            "branch": br(e.branch_candidate)} for e in trace.evaluations],
           "decisions": [{"node_id": d.node_id, "kind": d.kind, "reason": d.reason,
                          "children": list(d.child_node_ids), "branch": br(d.branch_candidate)}
                         for d in trace.decisions]}
    save(tag, trace=np.array(json.dumps(out)))


GOLDENS = [
    ("crown_c1", lambda t: golden_crown(wl.make_c1(), t, pre_rows=8)),
    ("crown_c3_b16", lambda t: golden_crown(wl.subset(wl.make_c3(), 16), t, pre_rows=2)),
    ("crown_c2_allint_b4", lambda t: golden_all_intermediate(wl.subset(wl.make_c2(), 4), t)),
    ("alpha_c4_b4", lambda t: golden_alpha_cnn(wl.subset(wl.make_c4(), 4), t)),
    ("bab_c5_d256", lambda t: golden_bab_batch(wl.subset(wl.make_c5(), 256), t)),
    ("crown_c1_mixed", lambda t: golden_crown(wl.make_c1(eps=0.001, label_mode="predicted"), t, pre_rows=8)),
    ("bab_c5d2_mixed", lambda t: golden_bab_batch(
        wl.subset(wl.make_c5(eps=0.004, depth=2, label_mode="predicted"), 256), t)),
    ("fused_linear", lambda t: golden_fused_region(t, "linear")),
    ("fused_conv2d", lambda t: golden_fused_region(t, "conv2d")),
    ("alpha_shared_mlp", golden_shared_alpha),
    ("task_ibp_c1_b8", lambda t: golden_task_ibp(wl.subset(wl.make_c1(), 8), t)),
    ("task_ibp_c3_b4", lambda t: golden_task_ibp(wl.subset(wl.make_c3(), 4), t)),
    ("task_ibp_dag", lambda t: golden_task_ibp(wl.make_ibp_dag(), t)),
    ("task_ibp_dag_box", lambda t: golden_task_ibp(wl.make_ibp_dag(box=True), t)),
    ("task_ibp_dag_sched", lambda t: golden_task_ibp_scheduled(wl.make_ibp_dag(), t)),
    ("bab_solve_ab_e003", golden_bab_solve),
    ("bab_solve_ab_e005", golden_bab_solve),
    ("bab_solve_alpha_e005", golden_bab_solve),
    ("bab_solve_cert_single", golden_bab_solve),
    ("bab_solve_cert_fallback", golden_bab_solve),
    ("bab_solve_cert_prune", golden_bab_solve),
    ("bab_solve_1d", golden_bab_solve),
    ("bab_solve_obj_both", golden_bab_solve),
    ("bab_solve_obj_alpha_gap", golden_bab_solve),
    ("bab_solve_cnn_b1", golden_bab_solve),
    ("bab_solve_cnn_b4", golden_bab_solve),
    ("cert_c3_conv", golden_cert_conv),
    ("lp_reference_p2", golden_lp),
    ("lp_reference_p1", golden_lp),
    ("frontend_planned", golden_frontend),
    ("vnnlib_queries", golden_vnnlib),
    ("objectives_mlp", golden_objectives),
    ("crown_c3_box", lambda t: golden_crown(c3_box(), t, pre_rows=6)),
] + [
    (f"crown_dag_{k}{'_box' if b else ''}", (lambda k, b: lambda t: golden_crown(dag_case(k, b), t))(k, b))
    for k in wl.DAG_KINDS for b in (False, True)
] + [
    ("alpha_crown_objectives", golden_alpha_crown_objectives),
    ("native_toy_b4", golden_native),
    ("native_toy_budget", golden_native),
    ("native_mlp", golden_native),
]


def main(argv) -> None:
    """Regenerate every fixture, or only those whose tag contains one of ``argv``."""
    torch.set_num_threads(8)
    for tag, make in GOLDENS:
        if not argv or any(a in tag for a in argv):
            make(tag)


if __name__ == "__main__":
    main(sys.argv[1:])
