"""CPU restatement of the reference IBP task executors (test infrastructure only).

Only tests, the smoke check and the bench's CPU baseline use this module, as
the checker; nothing in ``boundflow_amd`` imports it.

Follows op by op, with the same torch operations and association order:

* ``run_ibp`` -- PythonTaskExecutor.run_ibp, boundflow/runtime/task_executor.py:127-358
  (input set -> ``concretize_matmul`` for ``linear``, bounding box for every
  other op; W+/W- interval affine; c/r batched linear :228-244; spec_linear
  :185-213; add :266-280; mul = domains/interval.py:102-112; concat with
  runtime/dag_utils.py:6-47; flatten default start_dim 0 :312-320)
* ``run_ibp_task`` -- PythonTaskExecutor.run_ibp_task, task_executor.py:360-563
  (environment keyed by physical buffer id; interval operands, params
  included, resolved through the storage plan)
* ``run_ibp_scheduled`` -- boundflow/runtime/scheduler.py:160-255

Pinned by: the reference-generated fixtures ``task_ibp_*`` (tests/golden), and
in ``tests/test_oracle_task_ibp.py`` by soundness on sampled points, brute-force
interval products and the equality of the scheduled and single-task runs.
"""

from __future__ import annotations

from typing import Any, Dict, Optional

import torch

from boundflow_amd.ir import BFTaskModule, StoragePlan
from boundflow_amd.spec import BoxPerturbation, InputSpec, IntervalState, LpBallPerturbation, normalize_input_spec

from .crown_ref import _dual_row_norm, interval_affine


class _Ball:
    def __init__(self, spec: InputSpec):
        self.spec = spec


def _box(x) -> IntervalState:
    if isinstance(x, IntervalState):
        return x
    lo, hi = x.spec.perturbation.bounding_box(x.spec.center)
    return IntervalState(lo, hi)


def _concretize_matmul(spec: InputSpec, w: torch.Tensor, b) -> IntervalState:
    """perturbation.py:102-173 (Lp ball, rank-2 and rank-3 weights) and :282-325 (box)."""
    c = spec.center
    if c.dim() != 2:
        raise ValueError(f"concretize_matmul expects center rank-2 [B,I], got {tuple(c.shape)}")
    p = spec.perturbation
    if isinstance(p, LpBallPerturbation):
        eps = float(p.eps)
        q = p.normalized_p()
        if w.dim() == 2:
            out = c.matmul(w.t())
            dev = eps * _dual_row_norm(w, q, dim=1).unsqueeze(0)
        else:
            out = torch.bmm(c.unsqueeze(1), w.transpose(1, 2)).squeeze(1)
            dev = eps * _dual_row_norm(w, q, dim=2)
        lb, ub = out - dev, out + dev
    else:
        mid = (p.lower + p.upper) / 2.0
        rad = (p.upper - p.lower) / 2.0
        if w.dim() == 2:
            out = mid.matmul(w.t())
            dev = rad.matmul(w.abs().t())
        else:
            out = torch.bmm(mid.unsqueeze(1), w.transpose(1, 2)).squeeze(1)
            dev = torch.bmm(rad.unsqueeze(1), w.abs().transpose(1, 2)).squeeze(1)
        lb, ub = out - dev, out + dev
    if b is not None:
        lb, ub = lb + b, ub + b
    return IntervalState(lb, ub)


def _batched_linear(x: IntervalState, w: torch.Tensor, b) -> IntervalState:
    """task_executor.py:228-244."""
    if b is None:
        b = torch.as_tensor(0.0)
    mid = (x.lower + x.upper) / 2.0
    diff = (x.upper - x.lower) / 2.0
    center = torch.bmm(mid.unsqueeze(1), w.transpose(-1, -2)).squeeze(1)
    dev = torch.bmm(diff.unsqueeze(1), w.abs().transpose(-1, -2)).squeeze(1)
    return IntervalState(center - dev + b, center + dev + b)


def _spec_linear(x: IntervalState, C: torch.Tensor) -> IntervalState:
    if C.dim() != 3:
        raise ValueError(f"spec_linear expects C rank-3 [B,S,O], got {tuple(C.shape)}")
    cp, cn = torch.clamp(C, min=0.0), torch.clamp(C, max=0.0)
    l, u = x.lower.unsqueeze(1), x.upper.unsqueeze(1)
    return IntervalState((cp * l + cn * u).sum(dim=-1), (cp * u + cn * l).sum(dim=-1))


def _concat_axis(axis: int, rank: int) -> int:
    if (rank == 2 and axis in (1, -1)) or (rank == 4 and axis in (1, -3)):
        return 1
    raise NotImplementedError(f"concat axis {axis} on rank {rank}")


def _apply(op, get_state, get_tensor) -> Any:
    t = op.op_type
    if t == "spec_linear":
        return _spec_linear(_box(get_state(op.inputs[0])), get_tensor(op.inputs[1]))
    if t == "linear":
        x = get_state(op.inputs[0])
        w = get_tensor(op.inputs[1])
        b = get_tensor(op.inputs[2]) if len(op.inputs) == 3 else None
        if isinstance(x, _Ball):
            return _concretize_matmul(x.spec, w, b)
        if w.dim() == 3:
            return _batched_linear(x, w, b)
        lo, hi = interval_affine(x.lower, x.upper, w, b, {"op": "linear"})
        return IntervalState(lo, hi)
    if t == "conv2d":
        x = _box(get_state(op.inputs[0]))
        b = get_tensor(op.inputs[2]) if len(op.inputs) == 3 else None
        attrs = dict(op.attrs)
        attrs.setdefault("op", "conv2d")
        lo, hi = interval_affine(x.lower, x.upper, get_tensor(op.inputs[1]), b, attrs)
        return IntervalState(lo, hi)
    if t == "relu":
        x = _box(get_state(op.inputs[0]))
        return IntervalState(torch.relu(x.lower), torch.relu(x.upper))
    if t == "add":
        a, b = _box(get_state(op.inputs[0])), _box(get_state(op.inputs[1]))
        if a.lower.shape != b.lower.shape:
            raise NotImplementedError("add with exact same-shape inputs only")
        return IntervalState(a.lower + b.lower, a.upper + b.upper)
    if t == "mul":
        a, b = _box(get_state(op.inputs[0])), _box(get_state(op.inputs[1]))
        cand = torch.stack([a.lower * b.lower, a.lower * b.upper, a.upper * b.lower, a.upper * b.upper], dim=0)
        return IntervalState(cand.min(dim=0).values, cand.max(dim=0).values)
    if t == "concat":
        parts = [_box(get_state(n)) for n in op.inputs]
        axis = _concat_axis(int(op.attrs.get("axis", 1)), parts[0].lower.dim())
        return IntervalState(torch.cat([p.lower for p in parts], dim=axis),
                             torch.cat([p.upper for p in parts], dim=axis))
    if t == "flatten":
        x = _box(get_state(op.inputs[0]))
        sd, ed = int(op.attrs.get("start_dim", 0)), int(op.attrs.get("end_dim", -1))
        return IntervalState(torch.flatten(x.lower, sd, ed), torch.flatten(x.upper, sd, ed))
    if t == "reshape":
        x = _box(get_state(op.inputs[0]))
        shape = op.attrs.get("shape")
        return x if shape is None else IntervalState(x.lower.reshape(shape), x.upper.reshape(shape))
    if t in ("permute", "transpose"):
        x = _box(get_state(op.inputs[0]))
        dims = [int(d) for d in op.attrs["dims"]]
        return IntervalState(x.lower.permute(*dims), x.upper.permute(*dims))
    raise NotImplementedError(f"unsupported op_type: {t}")


def run_ibp(module: BFTaskModule, input_spec, *, output_value: Optional[str] = None) -> IntervalState:
    task = module.get_entry_task()
    spec = normalize_input_spec(input_spec)
    params = module.params
    env: Dict[str, Any] = {spec.value_name: _Ball(spec)}

    def get_state(name):
        if name in env:
            return env[name]
        t = params[name]
        return IntervalState(t, t)

    for op in task.ops:
        env[op.outputs[0]] = _apply(op, get_state, lambda n: params[n])
    return _box(env[output_value or task.output_values[0]])


def run_ibp_task(task, *, env: Dict[str, IntervalState], params: Dict[str, Any], storage_plan: StoragePlan) -> None:
    def buf(name):
        return storage_plan.to_physical(storage_plan.value_to_buffer[name])

    def get_state(name):
        bid = buf(name)
        if bid not in env:
            t = params[name]
            env[bid] = IntervalState(t, t)
        return env[bid]

    for op in task.ops:
        env[buf(op.outputs[0])] = _apply(op, get_state, lambda n: params[n])


def run_ibp_scheduled(module: BFTaskModule, input_spec, *, output_value: Optional[str] = None) -> IntervalState:
    spec = input_spec
    if isinstance(spec, InputSpec):
        if isinstance(spec.perturbation, BoxPerturbation) or spec.perturbation.normalized_p() != "inf":
            raise NotImplementedError("scheduled IBP takes Linf specifications")
        eps = float(spec.perturbation.eps)
    else:
        eps = float(spec.eps)
    plan = module.storage_plan
    x0 = spec.center
    env = {plan.to_physical(plan.value_to_buffer[spec.value_name]): IntervalState(x0 - eps, x0 + eps)}
    tasks = {t.task_id: t for t in module.tasks}
    graph = module.task_graph
    for tid in graph.topo_sort(tasks_by_id=tasks, entry_task_id=module.entry_task_id):
        run_ibp_task(tasks[tid], env=env, params=module.params, storage_plan=plan)
    if output_value is None:
        reach = graph.reachable_from(module.entry_task_id)
        srcs = {e.src_task_id for e in graph.edges if e.src_task_id in reach and e.dst_task_id in reach}
        (sink,) = [t for t in reach if t not in srcs]
        output_value = tasks[sink].output_values[0]
    return env[plan.to_physical(plan.value_to_buffer[output_value])]
