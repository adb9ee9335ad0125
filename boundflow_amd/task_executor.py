"""HIP IBP executor over planner BoundTasks and storage plans.

Drop-in counterpart of the reference's IBP executors:

* ``HipTaskExecutor.run_ibp`` -- ``TaskExecutor.run_ibp`` / ``PythonTaskExecutor.run_ibp``
  (boundflow/runtime/task_executor.py:108-358): single-task IBP from an input
  specification, with ``concretize_matmul`` semantics on the input layer.
* ``HipTaskExecutor.run_ibp_task`` -- ``IBPTaskStepExecutor.run_ibp_task``
  (boundflow/runtime/scheduler.py:21-30; PythonTaskExecutor
  task_executor.py:360-563; TVMTaskExecutor tvm_executor.py:592-728): one task on
  a shared environment keyed by *physical* buffer id through
  ``storage_plan.value_to_buffer`` -> ``to_physical``.
* ``run_ibp_scheduled`` -- boundflow/runtime/scheduler.py:160-255.

Unlike the reference's TVM executor, which copies every operand through host
numpy (tvm_executor.py:683-690), every tensor stays on the device and each op
is one HIP launch (linear/conv2d in center/radius form, relu, add, spec_linear,
batched linear); flatten/reshape are views.
"""

from __future__ import annotations

from typing import Any, Dict, Optional

import torch

from . import _lib
from .ir import BFTaskModule, BoundTask, StoragePlan, TaskKind
from .spec import (BoxPerturbation, InputSpec, IntervalState, LinfInputSpec, LpBallPerturbation, input_norm_p,
                   normalize_input_spec)


def _pair(v):
    if isinstance(v, int):
        return (v, v)
    v = tuple(int(x) for x in v)
    if len(v) == 1:
        return (v[0], v[0])
    if len(v) == 2:
        return v
    raise ValueError(f"invalid int tuple: {v} (expected dim=2)")


def _concat_axis(axis_raw, rank: int, caller: str) -> int:
    """Feature axis of [B, F] or channel axis of [B, C, H, W] (dag_utils.py:6-20)."""
    axis = int(axis_raw)
    if rank == 2 and axis in (1, -1):
        return 1
    if rank == 4 and axis in (1, -3):
        return 1
    if rank in (2, 4):
        raise NotImplementedError(f"{caller} only supports the feature/channel concat axis for rank {rank}, "
                                  f"got axis={axis}")
    raise NotImplementedError(f"{caller} only supports concat on rank-2 [B,F] or rank-4 [B,C,H,W], got rank={rank}")


def _check_concat_shapes(shapes, axis: int, caller: str) -> None:
    """Equal rank, equal non-axis dims (dag_utils.py:23-47)."""
    ref = tuple(shapes[0])
    for idx, shp in enumerate(shapes[1:], start=1):
        shp = tuple(shp)
        if len(shp) != len(ref):
            raise NotImplementedError(f"{caller} only supports concat with equal-rank inputs, got {ref} and {shp} "
                                      f"at input {idx}")
        if any(a != b for i, (a, b) in enumerate(zip(ref, shp)) if i != axis):
            raise NotImplementedError(f"{caller} only supports concat with exact same-shape non-axis dims, "
                                      f"got {ref} and {shp}")


class _InputBall:
    """The not-yet-concretized input set (task_executor.py:152-157)."""

    def __init__(self, spec: InputSpec):
        self.spec = spec


class HipTaskExecutor:
    """IBP over BoundTasks on the HIP device (backend replacing TVMTaskExecutor).

    Op semantics follow PythonTaskExecutor (task_executor.py:184-349): the input
    set reaches ``linear`` as the perturbation itself (``concretize_matmul``),
    every other op sees its bounding box; interval affine maps are computed in
    center/radius form (equal to the reference's W+/W- split up to fp32
    rounding of the summed terms).
    """

    # ---- op kernels -------------------------------------------------------
    def _linear_input(self, ball: _InputBall, w: torch.Tensor, b: Optional[torch.Tensor]) -> IntervalState:
        """``perturbation.concretize_matmul`` (perturbation.py:102-160)."""
        p = ball.spec.perturbation
        center = ball.spec.center
        if center.dim() != 2:
            raise ValueError(f"concretize_matmul expects center rank-2 [B,I], got {tuple(center.shape)}")
        B, K = (int(d) for d in center.shape)
        if w.dim() == 3:
            norm_p = input_norm_p(p)
            if norm_p == 0:
                # Linf ball or box: eps * sum |W| over the rows equals the bounding box's radius term
                lo, hi = p.bounding_box(center)
                return self._batched_linear(IntervalState(lo, hi), w, b)
            return self._batched_linear_ball(center, float(p.eps), norm_p, w, b)
        if int(w.shape[1]) != K:
            raise ValueError(f"matmul shape mismatch: center={tuple(center.shape)} weight={tuple(w.shape)}")
        if isinstance(p, BoxPerturbation):
            in_lo, in_hi, kind, eps = p.lower.reshape(B, K).contiguous(), p.upper.reshape(B, K).contiguous(), 0, 0.0
        else:
            # input kinds 1, 2, 3: Linf, L2, L1 ball (eps times the dual norm of each W row)
            kind = {0: 1, 2: 2, 1: 3}[input_norm_p(p)]
            in_lo, in_hi, eps = center.contiguous(), None, float(p.eps)
        return self._dense_linear(in_lo, in_hi, kind, eps, w, b)

    def _batched_linear_ball(self, center: torch.Tensor, eps: float, norm_p: int, w: torch.Tensor,
                             b: Optional[torch.Tensor]) -> IntervalState:
        """Per-sample weights W [B, O, I] over an L2 / L1 ball (perturbation.py:146-173): the
        rows of W[b] concretized against center[b] with the ball's dual norm
        (bf_concretize_dense: W[b, o] . c[b] -/+ eps * ||W[b, o]||_q + bias)."""
        B, O, I = (int(d) for d in w.shape)
        if tuple(center.shape) != (B, I):
            raise ValueError(f"batched matmul mismatch: center={tuple(center.shape)} weight={tuple(w.shape)}")
        dev = center.device
        rows = w.to(torch.float32).contiguous()
        bias = None if b is None else b.to(device=dev, dtype=torch.float32).expand(B, O).contiguous()
        lo = torch.empty(B, O, device=dev)
        hi = torch.empty_like(lo)
        c = center.to(torch.float32).contiguous()
        stream = _lib.stream_handle()
        for out, is_lower in ((lo, 1), (hi, 0)):
            _lib.call("bf_concretize_dense", _lib.ptr(rows), B, O, I, _lib.ptr(c), None, eps, norm_p, _lib.ptr(bias),
                      is_lower, _lib.ptr(out), stream)
        return IntervalState(lo, hi)

    def _dense_linear(self, in_lo, in_hi, kind: int, eps: float, w: torch.Tensor,
                      b: Optional[torch.Tensor]) -> IntervalState:
        B, K = (int(d) for d in in_lo.shape)
        N = int(w.shape[0])
        if int(w.shape[1]) != K:
            raise ValueError(f"linear shape mismatch: x={tuple(in_lo.shape)} weight={tuple(w.shape)}")
        dev = in_lo.device
        lo = torch.empty(B, N, device=dev)
        hi = torch.empty_like(lo)
        ws = torch.empty(int(_lib.load().bf_ibp_linear_workspace(B, K, N)), device=dev)
        _lib.call("bf_ibp_linear", _lib.ptr(in_lo), _lib.ptr(in_hi), B, K, kind, eps, 0, _lib.ptr(w.contiguous()),
                  _lib.ptr(None if b is None else b.contiguous()), N, None, 0, _lib.ptr(ws), _lib.ptr(lo),
                  _lib.ptr(hi), None, None, None, _lib.stream_handle())
        return IntervalState(lo, hi)

    def _batched_linear(self, iv: IntervalState, w: torch.Tensor, b: Optional[torch.Tensor]) -> IntervalState:
        """Per-sample weights W [B, O, I] (task_executor.py:228-244)."""
        B, O, I = (int(d) for d in w.shape)
        if tuple(iv.lower.shape) != (B, I):
            raise ValueError(f"batched linear shape mismatch: x={tuple(iv.lower.shape)} weight={tuple(w.shape)}")
        lo = torch.empty(B, O, device=w.device)
        hi = torch.empty_like(lo)
        bb = None if b is None else b.expand(B, O).contiguous()
        _lib.call("bf_ibp_batched_linear", _lib.ptr(iv.lower.contiguous()), _lib.ptr(iv.upper.contiguous()), B, I,
                  _lib.ptr(w.contiguous()), _lib.ptr(bb), O, _lib.ptr(lo), _lib.ptr(hi), _lib.stream_handle())
        return IntervalState(lo, hi)

    def _linear(self, x, w: torch.Tensor, b: Optional[torch.Tensor]) -> IntervalState:
        if isinstance(x, _InputBall):
            return self._linear_input(x, w, b)
        if w.dim() == 3:
            return self._batched_linear(x, w, b)
        lead = x.lower.shape[:-1]
        K = int(x.lower.shape[-1])
        out = self._dense_linear(x.lower.reshape(-1, K).contiguous(), x.upper.reshape(-1, K).contiguous(), 0, 0.0,
                                 w, b)
        N = int(w.shape[0])
        return IntervalState(out.lower.reshape(*lead, N), out.upper.reshape(*lead, N))

    def _conv(self, iv: IntervalState, w: torch.Tensor, b: Optional[torch.Tensor], attrs) -> IntervalState:
        if int(attrs.get("groups", 1)) != 1 or _pair(attrs.get("dilation", 1)) != (1, 1):
            raise NotImplementedError("HIP conv2d supports groups=1, dilation=1")
        B, Ci, Hi, Wi = (int(d) for d in iv.lower.shape)
        Co, KH, KW = int(w.shape[0]), int(w.shape[2]), int(w.shape[3])
        if int(w.shape[1]) != Ci:
            raise ValueError(f"conv2d channel mismatch: x={tuple(iv.lower.shape)} weight={tuple(w.shape)}")
        sh, sw = _pair(attrs.get("stride", 1))
        ph, pw = _pair(attrs.get("padding", 0))
        Ho = (Hi + 2 * ph - KH) // sh + 1
        Wo = (Wi + 2 * pw - KW) // sw + 1
        dev = iv.lower.device
        lo = torch.empty(B, Co, Ho, Wo, device=dev)
        hi = torch.empty_like(lo)
        ws = torch.empty(int(_lib.load().bf_ibp_conv2d_workspace(B, Ci * Hi * Wi, Co * Ho * Wo)), device=dev)
        _lib.call("bf_ibp_conv2d", _lib.ptr(iv.lower.contiguous()), _lib.ptr(iv.upper.contiguous()), B, Ci, Hi, Wi, 0,
                  0.0, 0, _lib.ptr(w.contiguous()), _lib.ptr(None if b is None else b.contiguous()), Co, KH, KW, sh,
                  sw, ph, pw, Ho, Wo, None, 0, _lib.ptr(ws), _lib.ptr(lo), _lib.ptr(hi), None, None,
                  _lib.stream_handle())
        return IntervalState(lo, hi)

    @staticmethod
    def _interval(x) -> IntervalState:
        """``ensure_interval`` (task_executor.py:169-178)."""
        if isinstance(x, IntervalState):
            return x
        if isinstance(x, _InputBall):
            lo, hi = x.spec.perturbation.bounding_box(x.spec.center)
            return IntervalState(lo, hi)
        raise TypeError(f"expected IntervalState or input perturbation, got {type(x)}")

    def _elementwise(self, name: str, a: IntervalState, b: IntervalState, shape) -> IntervalState:
        al, au = a.lower.expand(shape).contiguous(), a.upper.expand(shape).contiguous()
        bl, bu = b.lower.expand(shape).contiguous(), b.upper.expand(shape).contiguous()
        lo = torch.empty(shape, device=al.device)
        hi = torch.empty_like(lo)
        _lib.call(name, _lib.ptr(al), _lib.ptr(au), _lib.ptr(bl), _lib.ptr(bu), lo.numel(), _lib.ptr(lo),
                  _lib.ptr(hi), _lib.stream_handle())
        return IntervalState(lo, hi)

    def _relu(self, iv: IntervalState) -> IntervalState:
        lo = torch.empty(iv.lower.shape, device=iv.lower.device)
        hi = torch.empty_like(lo)
        _lib.call("bf_interval_relu", _lib.ptr(iv.lower.contiguous()), _lib.ptr(iv.upper.contiguous()),
                  lo.numel(), _lib.ptr(lo), _lib.ptr(hi), _lib.stream_handle())
        return IntervalState(lo, hi)

    def _spec_linear(self, iv: IntervalState, C: torch.Tensor, *, check_logits: bool) -> IntervalState:
        if C.dim() != 3:
            raise ValueError(f"spec_linear expects C rank-3 [B,S,O], got {tuple(C.shape)}")
        if check_logits:
            if iv.lower.dim() != 2:
                raise ValueError(f"spec_linear expects logits rank-2 [B,O], got {tuple(iv.lower.shape)}")
            if C.shape[0] != iv.lower.shape[0] or C.shape[2] != iv.lower.shape[1]:
                raise ValueError(f"spec_linear shape mismatch: C={tuple(C.shape)} logits={tuple(iv.lower.shape)}")
        B, S, O = (int(d) for d in C.shape)
        lo = torch.empty(B, S, device=C.device)
        hi = torch.empty_like(lo)
        _lib.call("bf_spec_linear", _lib.ptr(C.contiguous()), _lib.ptr(iv.lower.reshape(B, O).contiguous()),
                  _lib.ptr(iv.upper.reshape(B, O).contiguous()), B, S, O, _lib.ptr(lo), _lib.ptr(hi),
                  _lib.stream_handle())
        return IntervalState(lo, hi)

    def _apply(self, op, get_state, get_tensor, *, caller: str, check_logits: bool = True):
        t = op.op_type
        iv = lambda name: self._interval(get_state(name))  # noqa: E731
        if t == "spec_linear":
            return self._spec_linear(iv(op.inputs[0]), get_tensor(op.inputs[1]), check_logits=check_logits)
        if t == "linear":
            return self._linear(get_state(op.inputs[0]), get_tensor(op.inputs[1]),
                                get_tensor(op.inputs[2]) if len(op.inputs) == 3 else None)
        if t == "conv2d":
            return self._conv(iv(op.inputs[0]), get_tensor(op.inputs[1]),
                              get_tensor(op.inputs[2]) if len(op.inputs) == 3 else None, op.attrs)
        if t == "relu":
            return self._relu(iv(op.inputs[0]))
        if t == "add":
            a, b = iv(op.inputs[0]), iv(op.inputs[1])
            if tuple(a.lower.shape) != tuple(b.lower.shape) or tuple(a.upper.shape) != tuple(b.upper.shape):
                raise NotImplementedError(f"{caller} only supports add with exact same-shape inputs; "
                                          f"got {tuple(a.lower.shape)} and {tuple(b.lower.shape)}")
            return self._elementwise("bf_interval_add", a, b, a.lower.shape)
        if t == "mul":
            a, b = iv(op.inputs[0]), iv(op.inputs[1])
            shape = torch.broadcast_shapes(a.lower.shape, b.lower.shape)
            return self._elementwise("bf_interval_mul", a, b, shape)
        if t == "concat":
            if len(op.inputs) < 2:
                raise ValueError(f"concat expects at least 2 inputs, got {len(op.inputs)}")
            parts = [iv(name) for name in op.inputs]
            axis = _concat_axis(op.attrs.get("axis", 1), int(parts[0].lower.dim()), caller)
            _check_concat_shapes([tuple(p.lower.shape) for p in parts], axis, f"{caller} only supports concat")
            return IntervalState(torch.cat([p.lower for p in parts], dim=axis),
                                 torch.cat([p.upper for p in parts], dim=axis))
        if t == "flatten":
            x = iv(op.inputs[0])
            sd, ed = int(op.attrs.get("start_dim", 0)), int(op.attrs.get("end_dim", -1))
            return IntervalState(torch.flatten(x.lower, sd, ed), torch.flatten(x.upper, sd, ed))
        if t == "reshape":
            x = iv(op.inputs[0])
            shape = op.attrs.get("shape")
            if shape is None:
                return x
            return IntervalState(x.lower.reshape(shape), x.upper.reshape(shape))
        if t in ("permute", "transpose"):
            x = iv(op.inputs[0])
            dims = op.attrs.get("dims")
            if not isinstance(dims, (list, tuple)):
                raise ValueError(f"transpose missing dims for op '{op.name}': {dims}")
            dims = [int(d) for d in dims]
            return IntervalState(x.lower.permute(*dims), x.upper.permute(*dims))
        raise NotImplementedError(f"unsupported op_type in task executor: {t}")

    # ---- entry points -------------------------------------------------------
    def run_ibp(self, module: BFTaskModule, input_spec, *, output_value: Optional[str] = None) -> IntervalState:
        """task_executor.py:127-358."""
        module.validate()
        task = module.get_entry_task()
        if task.kind != TaskKind.INTERVAL_IBP:
            raise NotImplementedError(f"HipTaskExecutor only supports INTERVAL_IBP, got {task.kind}")
        spec = normalize_input_spec(input_spec)
        if spec.value_name not in task.input_values:
            raise ValueError(f"input_spec.value_name '{spec.value_name}' not in task.input_values: {task.input_values}")
        params = module.params
        env: Dict[str, Any] = {spec.value_name: _InputBall(spec)}

        def get_state(name):
            if name in env:
                return env[name]
            if name in params:
                t = params[name]
                return IntervalState(t, t)
            raise KeyError(f"missing value in env/params: {name}")

        def get_tensor(name):
            if name in params:
                return params[name]
            raise KeyError(f"missing param tensor: {name}")

        for op in task.ops:
            env[op.outputs[0]] = self._apply(op, get_state, get_tensor, caller="HipTaskExecutor.run_ibp")
        out = output_value or (task.output_values[0] if len(task.output_values) == 1 else None)
        if out is None:
            raise ValueError(f"task has {len(task.output_values)} outputs; specify output_value explicitly")
        return self._interval(env[out])

    def run_ibp_task(self, task: BoundTask, *, env: Dict[str, IntervalState], params: Dict[str, Any],
                     storage_plan: StoragePlan) -> None:
        """scheduler.py:21-30 / task_executor.py:360-563: mutate ``env`` (physical buffer id -> interval)."""
        if task.kind != TaskKind.INTERVAL_IBP:
            raise NotImplementedError(f"HipTaskExecutor only supports INTERVAL_IBP, got {task.kind}")

        def buf(value_name: str) -> str:
            logical = storage_plan.value_to_buffer.get(value_name)
            if logical is None:
                raise KeyError(f"value not found in storage_plan: {value_name}")
            phys = storage_plan.to_physical(logical)
            if storage_plan.physical_buffers and phys not in storage_plan.physical_buffers:
                raise KeyError(f"physical buffer_id not found in storage_plan.physical_buffers: {phys} (value={value_name})")
            return phys

        def get_state(name):
            bid = buf(name)
            if bid in env:
                return env[bid]
            if name in params:
                t = params[name]
                st = IntervalState(t, t)
                env[bid] = st
                return st
            raise KeyError(f"missing value in env/params: {name}")

        def get_tensor(name):
            if name in params:
                return params[name]
            raise KeyError(f"missing param tensor: {name}")

        for op in task.ops:
            env[buf(op.outputs[0])] = self._apply(op, get_state, get_tensor, caller="HipTaskExecutor.run_ibp_task",
                                                  check_logits=False)


def run_ibp_scheduled(module: BFTaskModule, input_spec, *, executor: Optional[HipTaskExecutor] = None,
                      output_value: Optional[str] = None) -> IntervalState:
    """Tasks of ``module.task_graph`` in topological order on one buffer
    environment (scheduler.py:160-255).  The input enters as the box
    ``x0 -+ eps`` of a Linf specification; modules without a task graph run
    as one task through ``run_ibp``."""
    module.validate()
    executor = executor or HipTaskExecutor()
    entry = module.get_entry_task()
    if entry.kind != TaskKind.INTERVAL_IBP:
        raise NotImplementedError(f"scheduler only supports INTERVAL_IBP, got {entry.kind}")
    spec = input_spec
    if isinstance(spec, InputSpec):
        p = spec.perturbation
        if isinstance(p, LpBallPerturbation) and p.normalized_p() == "inf":
            spec = LinfInputSpec(value_name=spec.value_name, center=spec.center, eps=float(p.eps))
        else:
            raise NotImplementedError("run_ibp_scheduled supports Linf input specifications only; "
                                      "use HipTaskExecutor.run_ibp for other perturbations")
    plan = module.storage_plan
    params = module.params

    def phys(value: str, what: str) -> str:
        logical = plan.value_to_buffer.get(value)
        if logical is None:
            raise KeyError(f"{what} not found in storage_plan: {value}")
        bid = plan.to_physical(logical)
        if plan.physical_buffers and bid not in plan.physical_buffers:
            raise KeyError(f"{what} physical buffer_id not found in storage_plan.physical_buffers: {bid}")
        return bid

    x0 = spec.center
    eps = float(spec.eps)
    in_phys = phys(spec.value_name, "input_spec.value_name")
    if module.task_graph is None:
        return executor.run_ibp(module, spec, output_value=output_value)
    # the input box, computed by the interval-add kernel as x0 + [-eps, +eps]
    neg = torch.full_like(x0, -eps)
    pos = torch.full_like(x0, eps)
    env: Dict[str, IntervalState] = {in_phys: executor._elementwise("bf_interval_add", IntervalState(x0, x0),
                                                                     IntervalState(neg, pos), x0.shape)}
    graph = module.task_graph
    tasks = {t.task_id: t for t in module.tasks}
    for task_id in graph.topo_sort(tasks_by_id=tasks, entry_task_id=module.entry_task_id):
        task = tasks[task_id]
        if task.kind != TaskKind.INTERVAL_IBP:
            raise NotImplementedError(f"mixed TaskKind not supported in the scheduler: {task.kind}")
        executor.run_ibp_task(task, env=env, params=params, storage_plan=plan)
    if output_value is None:
        reachable = graph.reachable_from(module.entry_task_id)
        out_deg = {t: 0 for t in reachable}
        for e in graph.edges:
            if e.src_task_id in reachable and e.dst_task_id in reachable:
                out_deg[e.src_task_id] += 1
        sinks = [t for t, d in out_deg.items() if d == 0]
        if len(sinks) != 1:
            raise ValueError(f"task_graph has {len(sinks)} sink tasks; specify output_value explicitly "
                             f"(sinks={sinks})")
        sink = tasks[sinks[0]]
        if len(sink.output_values) != 1:
            raise ValueError(f"sink task '{sink.task_id}' has {len(sink.output_values)} outputs; "
                             "specify output_value explicitly")
        output_value = sink.output_values[0]
    out_phys = phys(output_value, "output_value")
    if out_phys not in env and output_value in params:
        t = params[output_value]
        return IntervalState(t, t)
    if out_phys not in env:
        raise KeyError(f"missing output buffer in env: {out_phys} (value={output_value})")
    return env[out_phys]
