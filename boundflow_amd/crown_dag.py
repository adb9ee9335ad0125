"""CROWN-IBP on DAG networks (residual add, concat, fan-out) on the HIP path.

The reference's ``run_crown_ibp_mlp`` runs one general backward over any task
whose ops are linear / conv2d / relu / add / concat / flatten / reshape
(boundflow/runtime/crown_ibp.py:1669-2051): ops in reverse order, each popping
the backward state of its output, a value read by several ops accumulating
their contributions before its own op runs (:874-937), ``add`` handing the
same coefficient to every operand that depends on the input and folding a
constant operand into the bias (:1928-1970), ``concat`` handing each operand
its slice of the coefficient (:1972-2030).  ``crown.run_crown_ibp_mlp`` sends
every task that is not a chain here; chains keep the fused region kernels.

Layout: the backward state of a value is dense coefficient rows ``[M, n]``
(M = B * S, row m = domain m // S, spec m % S) for both bounds plus bias rows
``[M]``.  Each op is one or two HIP launches:

* linear -- ``bf_crown_relu_linear_fwd`` without a relaxation (A @ W and the bias
  rows, fp32 MFMA);
* conv2d -- ``bf_crown_relu_relax_lu`` without a relaxation (the bias rows) and
  ``bf_conv_transpose_rows``;
* relu -- ``bf_crown_relu_relax_lu`` (slopes from the pre-activation box, the
  optional lower-slope override and the lower-bound split coefficient);
* fan-in -- ``bf_interval_add`` over the two bounds' rows;
* concat -- a column slice of the rows per operand;
* the input -- ``bf_concretize_dense`` (Linf ball or box).

The forward trace is the op-by-op IBP of the reference's
``_forward_ibp_trace_mlp`` (crown_ibp.py:101-342) on the same kernels as the
chain trace, with ``bf_interval_relu`` / ``bf_interval_add`` for relu and add.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from types import SimpleNamespace
from typing import Dict, Mapping, Optional, Tuple

import torch

from . import _lib
from .conv import ibp_conv2d
from .ir import BFTaskModule, TaskKind
from .profiling import launch as _timed
from .spec import BoxPerturbation, InputSpec, IntervalState, LpBallPerturbation, input_norm_p, normalize_input_spec
from .task_executor import _check_concat_shapes, _concat_axis

DAG_OPS = ("linear", "conv2d", "relu", "add", "concat", "flatten", "reshape")


def _numel(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


def _pair(v) -> Tuple[int, int]:
    if isinstance(v, int):
        return (v, v)
    v = tuple(int(x) for x in v)
    return (v[0], v[0]) if len(v) == 1 else (v[0], v[1])


@dataclass
class DagTrace:
    """IBP boxes of every value, the (split/constraint-clipped) box of every ReLU
    input, and the per-sample shape of every value computed from the input."""
    interval_env: Dict[str, IntervalState]
    relu_pre: Dict[str, IntervalState]
    shapes: Dict[str, Tuple[int, ...]]
    # int32 [B]; None while no split or constraint was applied (no box can be emptied then):
    # ``infeasible`` makes the zeros on first read
    infeasible_flags: Optional[torch.Tensor] = None
    input_views: Dict[str, str] = field(default_factory=dict)   # value -> "input" for the input and its reshapes
    batch: int = 0
    device: Optional[torch.device] = None

    @property
    def infeasible(self) -> torch.Tensor:
        if self.infeasible_flags is None:
            self.infeasible_flags = torch.zeros(self.batch, dtype=torch.int32, device=self.device)
        return self.infeasible_flags


@dataclass
class _Rows:
    """Backward state of one value: coefficient rows of both bounds and their bias rows
    (None for a bound that is not computed)."""
    A_u: Optional[torch.Tensor]   # [M, n]
    A_l: Optional[torch.Tensor]   # [M, n] (may be the same tensor as A_u)
    b_u: Optional[torch.Tensor]   # [M]
    b_l: Optional[torch.Tensor]   # [M]


def _conv_geometry(op, W, in_shape):
    stride = _pair(op.attrs.get("stride", 1))
    padding = _pair(op.attrs.get("padding", 0))
    dilation = _pair(op.attrs.get("dilation", 1))
    if int(op.attrs.get("groups", 1)) != 1 or dilation != (1, 1):
        raise NotImplementedError("HIP conv2d supports groups=1, dilation=1")
    if len(in_shape) != 3 or in_shape[0] != int(W.shape[1]):
        raise ValueError(f"conv2d {op.name}: input shape {in_shape} vs weight {tuple(W.shape)}")
    kh, kw = int(W.shape[2]), int(W.shape[3])
    ho = (in_shape[1] + 2 * padding[0] - kh) // stride[0] + 1
    wo = (in_shape[2] + 2 * padding[1] - kw) // stride[1] + 1
    return stride, padding, (int(W.shape[0]), ho, wo)


def _conv_bias_map(bias: torch.Tensor, out_shape) -> torch.Tensor:
    """The per-channel bias of a conv layer as one value per output element."""
    Co, Ho, Wo = out_shape
    return bias.reshape(Co, 1).expand(Co, Ho * Wo).reshape(Co * Ho * Wo).contiguous()


def _module_task(module: BFTaskModule):
    module.validate()
    task = module.get_entry_task()
    if task.kind != TaskKind.INTERVAL_IBP:
        raise NotImplementedError(f"HIP CROWN only supports INTERVAL_IBP, got {task.kind}")
    if module.task_graph is not None or len(module.tasks) != 1:
        raise NotImplementedError("HIP CROWN supports single-task modules only")
    for op in task.ops:
        if len(op.outputs) != 1:
            raise NotImplementedError(f"HIP CROWN expects single-output ops, got outputs={op.outputs}")
        if op.op_type not in DAG_OPS:
            raise NotImplementedError(f"HIP CROWN: unsupported op_type {op.op_type}")
    return task


def relu_input_shapes(module: BFTaskModule, spec: InputSpec) -> Dict[str, Tuple[int, ...]]:
    """Per-sample shape of every ReLU input, in op order (the order of a trace's relu_pre),
    from the ops' shape rules alone (no launch)."""
    return value_shapes(module, spec)[1]


def value_shapes(module: BFTaskModule, spec: InputSpec):
    """Per-sample shapes of every value the ops compute (and the input), and of every
    ReLU input in op order, from the ops' shape rules alone (no launch)."""
    task = _module_task(module)
    params = module.params
    shapes: Dict[str, Tuple[int, ...]] = {spec.value_name: tuple(int(d) for d in spec.center.shape[1:])}

    def shape_of(name):
        return shapes[name] if name in shapes else tuple(int(d) for d in params[name].shape[1:])

    out: Dict[str, Tuple[int, ...]] = {}
    for op in task.ops:
        t = op.op_type
        x = op.inputs[0]
        if t == "linear":
            y = (int(params[op.inputs[1]].shape[0]),)
        elif t == "conv2d":
            y = _conv_geometry(op, params[op.inputs[1]], shape_of(x))[2]
        elif t == "relu":
            out[x] = shape_of(x)
            y = shape_of(x)
        elif t == "add":
            y = shape_of(x)
        elif t == "concat":
            parts = [shape_of(n) for n in op.inputs]
            y = (sum(p[0] for p in parts),) + tuple(parts[0][1:])
        elif t == "flatten":
            y = (_numel(shape_of(x)),)
        else:
            y = tuple(int(d) for d in op.attrs["shape"][1:])
        shapes[op.outputs[0]] = y
    return shapes, out


def forward_ibp_trace_dag(
    module: BFTaskModule,
    input_spec,
    *,
    relu_split_state: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_constraints: Optional[Mapping[str, IntervalState]] = None,
    raise_on_infeasible: bool = True,
) -> DagTrace:
    """Op-by-op IBP of crown_ibp.py:101-342 over a DAG task."""
    from .crown import _broadcast_split

    spec = normalize_input_spec(input_spec)
    task = _module_task(module)
    params = module.params
    center = spec.center
    _lib.require_device(center, "input center")
    B = int(center.shape[0])
    dev = center.device
    stream = _lib.stream_handle()
    pert = spec.perturbation
    box = isinstance(pert, BoxPerturbation)
    # a linear layer on the input takes the ball's dual row norm of W; every other consumer of
    # the input reads its bounding box (center -/+ eps for p = 1, 2, inf), as crown_ibp.py:125-178
    ibp_kind = 0 if box else {0: 1, 2: 2, 1: 3}[input_norm_p(pert)]
    # flags only where a split or a constraint can empty a box (the kernels take NULL)
    may_empty = bool(relu_split_state) or relu_pre_constraints is not None
    infeasible = torch.zeros(B, dtype=torch.int32, device=dev) if may_empty else None
    env: Dict[str, IntervalState] = {}
    relu_pre: Dict[str, IntervalState] = {}
    shapes: Dict[str, Tuple[int, ...]] = {spec.value_name: tuple(int(d) for d in center.shape[1:])}
    # the input set itself and its reshapes: (center, box lower, box upper) with the value's shape
    views: Dict[str, Tuple[torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor]]] = {
        spec.value_name: (center, pert.lower if box else None, pert.upper if box else None)}

    def box_of(name: str) -> IntervalState:
        if name in env:
            return env[name]
        if name in views:
            c, lo, hi = views[name]
            if lo is None:
                lo, hi = pert.bounding_box(c)
            return IntervalState(lo.contiguous(), hi.contiguous())
        if name in params:
            t = params[name].to(device=dev, dtype=torch.float32).contiguous()
            return IntervalState(t, t)
        raise KeyError(f"missing value in env/params: {name}")

    for op in task.ops:
        t = op.op_type
        out = op.outputs[0]
        x = op.inputs[0]
        if t == "linear":
            W = params[op.inputs[1]].contiguous()
            b = params[op.inputs[2]].contiguous() if len(op.inputs) == 3 else None
            if W.dim() != 2:
                raise NotImplementedError("batched linear weights are not supported")
            K, N = int(W.shape[1]), int(W.shape[0])
            if _numel(shapes[x] if x in shapes else box_of(x).lower.shape[1:]) != K:
                raise ValueError(f"linear {op.name}: input {x} does not have {K} features")
            lo = torch.empty(B, N, device=dev, dtype=torch.float32)
            hi = torch.empty_like(lo)
            ws = torch.empty(int(_lib.load().bf_ibp_linear_workspace(B, K, N)), device=dev, dtype=torch.float32)
            if x in views:
                c, blo, bhi = views[x]
                if box:
                    args = (blo.reshape(B, K).contiguous(), bhi.reshape(B, K).contiguous(), 0, 0.0)
                else:
                    args = (c.reshape(B, K).contiguous(), None, ibp_kind, float(pert.eps))
            else:
                xi = box_of(x)
                args = (xi.lower.reshape(B, K), xi.upper.reshape(B, K), 0, 0.0)
            _lib.call("bf_ibp_linear", _lib.ptr(args[0]), _lib.ptr(args[1]), B, K, args[2], args[3], 0, _lib.ptr(W),
                      _lib.ptr(b), N, None, 0, _lib.ptr(ws), _lib.ptr(lo), _lib.ptr(hi), None,
                      _lib.ptr(infeasible), None, stream)
            y = IntervalState(lo, hi)
            shapes[out] = (N,)
        elif t == "conv2d":
            W = params[op.inputs[1]].contiguous()
            b = params[op.inputs[2]].contiguous() if len(op.inputs) == 3 else None
            in_shape = shapes[x] if x in shapes else tuple(box_of(x).lower.shape[1:])
            stride, padding, out_shape = _conv_geometry(op, W, in_shape)
            layer = SimpleNamespace(weight=W, bias=b, in_shape=tuple(in_shape), out_shape=out_shape,
                                    attrs={"stride": stride, "padding": padding})
            lo = torch.empty((B,) + out_shape, device=dev, dtype=torch.float32)
            hi = torch.empty_like(lo)
            if x in views and not box:
                ibp_conv2d(views[x][0].contiguous(), None, 0, layer, None, 0, lo, hi, infeasible,
                           linf_eps=float(pert.eps))
            else:
                xi = box_of(x)
                ibp_conv2d(xi.lower.contiguous(), xi.upper.contiguous(), 0, layer, None, 0, lo, hi, infeasible)
            y = IntervalState(lo, hi)
            shapes[out] = out_shape
        elif t == "relu":
            xi = box_of(x)
            n = _numel(xi.lower.shape[1:])
            split = None
            split_ld = 0
            if relu_split_state is not None and x in relu_split_state:
                split, split_ld = _broadcast_split(relu_split_state[x].to(dev), B, n)
            constraint = relu_pre_constraints.get(x) if relu_pre_constraints is not None else None
            pre = xi
            if split is not None or constraint is not None:
                # the clipped box is the ReLU's own; other readers of x keep the IBP box
                pre = IntervalState(xi.lower.clone(), xi.upper.clone())
                _lib.call("bf_interval_clip", _lib.ptr(pre.lower), _lib.ptr(pre.upper),
                          _lib.ptr(None if constraint is None else constraint.lower.contiguous()),
                          _lib.ptr(None if constraint is None else constraint.upper.contiguous()),
                          _lib.ptr(split), split_ld, B, n, _lib.ptr(infeasible), stream)
            relu_pre[x] = pre
            lo = torch.empty_like(pre.lower)
            hi = torch.empty_like(pre.upper)
            _lib.call("bf_interval_relu", _lib.ptr(pre.lower), _lib.ptr(pre.upper), B * n, _lib.ptr(lo),
                      _lib.ptr(hi), stream)
            y = IntervalState(lo, hi)
            shapes[out] = tuple(int(d) for d in lo.shape[1:])
        elif t == "add":
            a, b2 = box_of(op.inputs[0]), box_of(op.inputs[1])
            if tuple(a.lower.shape) != tuple(b2.lower.shape):
                raise NotImplementedError(
                    "_forward_ibp_trace_mlp only supports add with exact same-shape inputs; "
                    f"got {tuple(a.lower.shape)} and {tuple(b2.lower.shape)}")
            lo = torch.empty_like(a.lower)
            hi = torch.empty_like(a.upper)
            _lib.call("bf_interval_add", _lib.ptr(a.lower), _lib.ptr(a.upper), _lib.ptr(b2.lower), _lib.ptr(b2.upper),
                      a.lower.numel(), _lib.ptr(lo), _lib.ptr(hi), stream)
            y = IntervalState(lo, hi)
            shapes[out] = tuple(int(d) for d in lo.shape[1:])
        elif t == "concat":
            if len(op.inputs) < 2:
                raise ValueError(f"concat expects at least 2 inputs, got {len(op.inputs)}")
            parts = [box_of(name) for name in op.inputs]
            axis = _concat_axis(op.attrs.get("axis", 1), int(parts[0].lower.dim()), "_forward_ibp_trace_mlp")
            _check_concat_shapes([tuple(p.lower.shape) for p in parts], axis, "_forward_ibp_trace_mlp")
            y = IntervalState(torch.cat([p.lower for p in parts], dim=axis),
                              torch.cat([p.upper for p in parts], dim=axis))
            shapes[out] = tuple(int(d) for d in y.lower.shape[1:])
        else:   # flatten / reshape
            if t == "flatten":
                if int(op.attrs.get("start_dim", 1)) != 1 or int(op.attrs.get("end_dim", -1)) != -1:
                    raise NotImplementedError("flatten(start_dim=1, end_dim=-1) only")
                new_shape = (B, -1)
            else:
                if "shape" not in op.attrs:
                    raise ValueError("reshape requires non-empty attrs['shape']")
                new_shape = tuple(int(d) for d in op.attrs["shape"])
            if x in views:
                c, blo, bhi = views[x]
                views[out] = (c.reshape(new_shape), None if blo is None else blo.reshape(new_shape),
                              None if bhi is None else bhi.reshape(new_shape))
                shapes[out] = tuple(int(d) for d in views[out][0].shape[1:])
                if box:
                    env[out] = IntervalState(views[out][1], views[out][2])
                continue
            xi = box_of(x)
            y = IntervalState(xi.lower.reshape(new_shape), xi.upper.reshape(new_shape))
            shapes[out] = tuple(int(d) for d in y.lower.shape[1:])
        env[out] = y
    if raise_on_infeasible and (relu_split_state or relu_pre_constraints):
        if bool(infeasible.any().item()):
            raise ValueError("infeasible relu split or constraint: lower>upper after applying split")
    return DagTrace(interval_env=env, relu_pre=relu_pre, shapes=shapes, infeasible_flags=infeasible, batch=B, device=dev,
                    input_views={name: spec.value_name for name in views})


def crown_backward_dag(
    module: BFTaskModule,
    spec: InputSpec,
    trace: DagTrace,
    *,
    linear_spec_C: Optional[torch.Tensor] = None,
    output_value: Optional[str] = None,
    relu_alpha: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_add_coeff_l: Optional[Dict[str, torch.Tensor]] = None,
    need_upper: bool = True,
    need_lower: bool = True,
    save: Optional[dict] = None,
    relu_influence: Optional[Dict[str, torch.Tensor]] = None,
) -> IntervalState:
    """The general backward of crown_ibp.py:1669-2051 on dense coefficient rows.  A bound
    that is not needed is not computed (its side of the result is None).  With ``save``
    (lower bound only) the coefficient entering every ReLU and the input's coefficient are
    kept for ``lower_grad_pass``.  With ``relu_influence`` each ReLU input x reached by the
    backward gets max over specs of max(|A_u|, |A_l|) of the coefficient of the ReLU's
    output, [B, *shape of x] (crown_ibp.py:1810-1833)."""
    from .crown import _flat_param, _init_spec, transposed

    task = _module_task(module)
    params = module.params
    dev = spec.center.device
    B = int(spec.center.shape[0])
    stream = _lib.stream_handle()
    if output_value is None:
        if len(task.output_values) != 1:
            raise ValueError(f"task has {len(task.output_values)} outputs; specify output_value explicitly")
        output_value = task.output_values[0]
    if output_value not in trace.shapes:
        raise ValueError(f"output_value {output_value} not produced by the task")
    if not (need_upper or need_lower):
        raise ValueError("crown_backward_dag: no bound requested")
    if save is not None and need_upper:
        raise ValueError("crown_backward_dag: the gradient pass follows the lower bound alone")
    out_dim = _numel(trace.shapes[output_value])
    A0, S, a_dstride = _init_spec(linear_spec_C, B, out_dim, dev)
    M = B * S
    if a_dstride == 0:
        A0 = A0.reshape(1, S, out_dim).expand(B, S, out_dim)
    A0 = A0.reshape(M, out_dim).contiguous()
    zero_b = torch.zeros(M, device=dev, dtype=torch.float32)
    adjoints: Dict[str, _Rows] = {output_value: _Rows(A0 if need_upper else None, A0 if need_lower else None,
                                                      zero_b if need_upper else None,
                                                      zero_b if need_lower else None)}
    dynamic = set(trace.shapes.keys())     # every value computed from the input (crown_ibp.py:912-919)
    if save is not None:
        save.update({"relu_A": {}, "ran": set(), "S": S, "output_value": output_value})

    def ptr_of(t):
        return None if t is None else t.data_ptr()

    def shared(st: _Rows) -> bool:
        """Both bounds carry the same rows (the spec itself, until the first ReLU splits them)."""
        return st.A_u is not None and st.A_l is not None and st.A_u.data_ptr() == st.A_l.data_ptr() \
            and st.b_u.data_ptr() == st.b_l.data_ptr()

    def like(st: _Rows, cols: int, one: bool):
        """Fresh (A_u, A_l) of [M, cols] for the bounds st carries (one buffer when shared)."""
        au = torch.empty(M, cols, device=dev) if st.A_u is not None else None
        al = (au if one else torch.empty(M, cols, device=dev)) if st.A_l is not None else None
        return au, al

    def zeros_like_b(st: _Rows):
        # bias rows are values (every step writes fresh ones): one zero row serves them all
        return (zero_b if st.b_u is not None else None), (zero_b if st.b_l is not None else None)

    def rows_pass(st: _Rows, n: int, *, pre=None, alpha=None, alpha_ld=0, add=None, add_ld=0, kbias=None,
                  cvec=None, name="crown_relu_relax"):
        """bf_crown_relu_relax_lu over the bounds st carries: (A', b + sums, center sums).  Without a
        relaxation, rows shared by both bounds are passed once."""
        one = pre is None and add is None and shared(st)
        rA_u, rA_l = like(st, n, one)
        nb_u, nb_l = like(_Rows(st.b_u, st.b_l, None, None), 1, one)
        nb_u = None if nb_u is None else nb_u.reshape(M)
        nb_l = None if nb_l is None else nb_l.reshape(M)
        c_u = torch.empty(M, device=dev) if (cvec is not None and st.A_u is not None) else None
        c_l = (c_u if one else torch.empty(M, device=dev)) if (cvec is not None and st.A_l is not None) else None
        A_l_in = None if one else st.A_l
        nz = int(st.A_u is not None) + int(A_l_in is not None)
        reads = 1 if (nz == 2 and ptr_of(st.A_u) == ptr_of(st.A_l)) else nz
        with _timed(name, 0.0, 4.0 * (reads + nz) * M * n):
            _lib.call("bf_crown_relu_relax_lu", _lib.ptr(st.A_u), _lib.ptr(A_l_in), S * n, B, S, n,
                      _lib.ptr(None if pre is None else pre.lower.reshape(B, n)),
                      _lib.ptr(None if pre is None else pre.upper.reshape(B, n)), _lib.ptr(alpha), alpha_ld,
                      _lib.ptr(add if A_l_in is not None else None), add_ld, _lib.ptr(kbias), _lib.ptr(cvec),
                      _lib.ptr(st.b_u), _lib.ptr(None if one else st.b_l), _lib.ptr(rA_u),
                      _lib.ptr(None if one else rA_l), _lib.ptr(nb_u), _lib.ptr(None if one else nb_l),
                      _lib.ptr(c_u), _lib.ptr(None if one else c_l), stream)
        return _Rows(rA_u, rA_l, nb_u, nb_l), (c_u, c_l)

    def add_rows(a, b, cols):
        if a is None:
            return None
        out = torch.empty(M, cols, device=dev) if cols > 1 else torch.empty(M, device=dev)
        _lib.call("bf_rows_add", _lib.ptr(a), _lib.ptr(b), M, cols, S, None, None, 0, _lib.ptr(out), stream)
        return out

    def accumulate(name: str, upd: _Rows) -> None:
        """crown_ibp.py:892-909: current + update, coefficients and bias rows."""
        cur = adjoints.get(name)
        if cur is None:
            adjoints[name] = upd
            return
        n = int((upd.A_u if upd.A_u is not None else upd.A_l).shape[1])
        both = shared(cur) and shared(upd)
        with _timed("dag_accumulate", 0.0, 4.0 * 3 * M * n * (1 if both else 2)):
            A_u = add_rows(cur.A_u, upd.A_u, n)
            A_l = A_u if both else add_rows(cur.A_l, upd.A_l, n)
        b_u = add_rows(cur.b_u, upd.b_u, 1)
        b_l = b_u if both else add_rows(cur.b_l, upd.b_l, 1)
        adjoints[name] = _Rows(A_u, A_l, b_u, b_l)

    for op_index in range(len(task.ops) - 1, -1, -1):
        op = task.ops[op_index]
        out = op.outputs[0]
        st = adjoints.pop(out, None)
        if st is None:
            continue
        if save is not None:
            save["ran"].add(op_index)
        t = op.op_type
        x = op.inputs[0]
        if t == "linear":
            W = params[op.inputs[1]].contiguous()
            bias = params[op.inputs[2]].contiguous() if len(op.inputs) == 3 else None
            N, P = int(W.shape[0]), int(W.shape[1])
            Wt = transposed(W)   # the contraction reads W^T [P, N]: 128-bit operand loads along N
            one = shared(st)
            nA_u, nA_l = like(st, P, one)
            nb_u, nb_l = like(_Rows(st.b_u, st.b_l, None, None), 1, one)
            nb_u = None if nb_u is None else nb_u.reshape(M)
            nb_l = None if nb_l is None else nb_l.reshape(M)
            A_l_in = None if one else st.A_l
            nz = int(st.A_u is not None) + int(A_l_in is not None)
            with _timed("crown_linear", 2.0 * nz * M * N * P, 4.0 * nz * (M * N + N * P + M * P)):
                _lib.call("bf_crown_relu_linear_fwd", _lib.ptr(st.A_u), _lib.ptr(A_l_in), S * N, B, S, N, None,
                          None, 0, _lib.ptr(Wt), P, 1, _lib.ptr(bias), _lib.ptr(st.b_u),
                          _lib.ptr(None if one else st.b_l), _lib.ptr(nA_u), _lib.ptr(None if one else nA_l),
                          _lib.ptr(nb_u), _lib.ptr(None if one else nb_l), stream)
            accumulate(x, _Rows(nA_u, nA_l, nb_u, nb_l))
        elif t == "conv2d":
            W = params[op.inputs[1]].contiguous()
            in_shape = trace.shapes[x]
            (sh, sw), (ph, pw), out_shape = _conv_geometry(op, W, in_shape)
            Co, Ho, Wo = out_shape
            Ci, Hi, Wi = in_shape
            n_out = Co * Ho * Wo
            if len(op.inputs) == 3:
                st, _ = rows_pass(st, n_out, kbias=_conv_bias_map(params[op.inputs[2]], out_shape),
                                  name="conv_bias_rows")
            one = shared(st)
            y_u, y_l = like(st, Ci * Hi * Wi, one)
            A_l_in = None if one else st.A_l
            nz = int(st.A_u is not None) + int(A_l_in is not None)
            KH, KW = int(W.shape[2]), int(W.shape[3])
            flops = 2.0 * nz * M * Ci * Hi * Wi * Co * KH * KW / float(sh * sw)
            with _timed("conv_transpose", flops, 4.0 * nz * (M * n_out + M * Ci * Hi * Wi)):
                _lib.call("bf_conv_transpose_rows", _lib.ptr(st.A_u), _lib.ptr(A_l_in), M, Co, Ho, Wo, _lib.ptr(W),
                          Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, _lib.ptr(y_u), _lib.ptr(None if one else y_l), S, None,
                          0, 0, None, None, None, None, stream)
            accumulate(x, _Rows(y_u, y_l, st.b_u, st.b_l))
        elif t == "relu":
            pre = trace.relu_pre[x]
            n = _numel(pre.lower.shape[1:])
            alpha = add = None
            alpha_ld = add_ld = 0
            if relu_alpha is not None and x in relu_alpha:
                alpha, alpha_ld = _flat_param(relu_alpha[x], B, n, f"relu_alpha[{x}]")
            if relu_pre_add_coeff_l is not None and x in relu_pre_add_coeff_l:
                add, add_ld = _flat_param(relu_pre_add_coeff_l[x], B, n, f"relu_pre_add_coeff_l[{x}]")
            if relu_influence is not None:
                if x in relu_influence:
                    raise ValueError(f"duplicate ReLU objective influence identity: {x}")
                infl = torch.empty((B,) + tuple(pre.lower.shape[1:]), device=dev, dtype=torch.float32)
                _lib.call("bf_rows_abs_max", _lib.ptr(st.A_u), _lib.ptr(st.A_l), B, S, n, _lib.ptr(infl), stream)
                relu_influence[x] = infl
            if save is not None:
                save["relu_A"][op_index] = st.A_l      # the coefficient before the relaxation
            new, _ = rows_pass(st, n, pre=pre, alpha=alpha, alpha_ld=alpha_ld, add=add, add_ld=add_ld)
            accumulate(x, new)
        elif t in ("flatten", "reshape"):
            accumulate(x, st)          # the rows are already laid out in the input's element order
        elif t == "add":
            out_shape = trace.shapes[out]
            n = _numel(out_shape)
            cb_u, cb_l = st.b_u, st.b_l
            dyn = []
            for name in op.inputs:
                if name in dynamic:
                    shp = trace.shapes[name]
                    val = None
                else:
                    val = params[name].to(device=dev, dtype=torch.float32)
                    shp = tuple(int(d) for d in val.shape[1:])
                if tuple(shp) != tuple(out_shape):
                    raise NotImplementedError(
                        f"run_crown_ibp_mlp only supports add with exact same-shape non-broadcast inputs; "
                        f"got output_shape={out_shape} input_shape={tuple(shp)}")
                if val is None:
                    dyn.append(name)
                    continue
                # a constant operand: its contribution sum_k A[m, k] * val[d, k] joins the bias
                if int(val.shape[0]) != B:
                    raise NotImplementedError(f"add operand {name}: expected a [B, ...] tensor, got {tuple(val.shape)}")
                zu, zl = zeros_like_b(st)
                _, (c_u, c_l) = rows_pass(_Rows(st.A_u, st.A_l, zu, zl), n, cvec=val.reshape(B, n).contiguous(),
                                          name="add_constant_rows")
                one = shared(st)
                cb_u = add_rows(cb_u, c_u, 1)
                cb_l = cb_u if one else add_rows(cb_l, c_l, 1)
            for idx, name in enumerate(dyn):
                # the bias goes with the first operand that depends on the input (crown_ibp.py:922-937)
                if idx == 0:
                    bu, bl = cb_u, cb_l
                else:
                    bu, bl = zeros_like_b(st)
                accumulate(name, _Rows(st.A_u, st.A_l, bu, bl))
        elif t == "concat":
            out_shape = trace.shapes[out]
            _concat_axis(op.attrs.get("axis", 1), len(out_shape) + 1, "run_crown_ibp_mlp")
            shapes = [trace.shapes[name] if name in dynamic else None for name in op.inputs]
            for name, shp in zip(op.inputs, shapes):
                if shp is None:
                    raise NotImplementedError(f"run_crown_ibp_mlp only supports concat over dynamic tensor values, "
                                              f"got {name}")
            _check_concat_shapes([(0,) + tuple(s) for s in shapes], 1, "run_crown_ibp_mlp")
            inner = _numel(out_shape[1:])
            one = shared(st)
            start = 0
            for idx, (name, shp) in enumerate(zip(op.inputs, shapes)):
                stop = start + int(shp[0])
                cols = slice(start * inner, stop * inner)
                A_u = st.A_u[:, cols].contiguous() if st.A_u is not None else None
                A_l = (A_u if one else st.A_l[:, cols].contiguous()) if st.A_l is not None else None
                if idx == 0:
                    bu, bl = st.b_u, st.b_l
                else:
                    bu, bl = zeros_like_b(st)
                accumulate(name, _Rows(A_u, A_l, bu, bl))
                start = stop
            if start != int(out_shape[0]):
                raise ValueError(f"run_crown_ibp_mlp concat backward shape mismatch: sliced={start} "
                                 f"output axis size is {int(out_shape[0])}")
        else:
            raise NotImplementedError(f"run_crown_ibp_mlp unsupported op_type in backward: {t}")

    st = adjoints.get(spec.value_name)
    if st is None:
        raise RuntimeError(f"run_crown_ibp_mlp backward did not reach input value {spec.value_name}")
    if save is not None:
        save["input_A"] = st.A_l
    return _concretize(spec, st, B, S)


def _input_center_radius(spec: InputSpec, B: int, I: int):
    """(center, rad or None, eps) of the input set: a box's midpoint and radius, or a Linf ball."""
    pert = spec.perturbation
    if isinstance(pert, BoxPerturbation):
        lo = pert.lower.reshape(B, I)
        hi = pert.upper.reshape(B, I)
        return ((lo + hi) / 2.0).contiguous(), ((hi - lo) / 2.0).contiguous(), 1.0
    return spec.center.reshape(B, I).contiguous(), None, float(pert.eps)


def _concretize(spec: InputSpec, st: _Rows, B: int, S: int) -> IntervalState:
    """concretize_affine (perturbation.py:175-222, 327-359) on dense rows."""
    stream = _lib.stream_handle()
    dev = spec.center.device
    I = int((st.A_u if st.A_u is not None else st.A_l).shape[1])
    center, rad, eps = _input_center_radius(spec, B, I)
    lb = torch.empty(B, S, device=dev) if st.A_l is not None else None
    ub = torch.empty(B, S, device=dev) if st.A_u is not None else None
    nz = int(lb is not None) + int(ub is not None)
    with _timed("concretize_dense", 2.0 * nz * B * S * I, 4.0 * nz * B * S * I):
        if ub is not None:
            _lib.call("bf_concretize_dense", _lib.ptr(st.A_u), B, S, I, _lib.ptr(center), _lib.ptr(rad), eps,
                      input_norm_p(spec.perturbation), _lib.ptr(st.b_u), 0, _lib.ptr(ub), stream)
        if lb is not None:
            _lib.call("bf_concretize_dense", _lib.ptr(st.A_l), B, S, I, _lib.ptr(center), _lib.ptr(rad), eps,
                      input_norm_p(spec.perturbation), _lib.ptr(st.b_l), 1, _lib.ptr(lb), stream)
    return IntervalState(lower=lb, upper=ub)


def lower_grad_pass(module: BFTaskModule, spec: InputSpec, trace: DagTrace, saved: dict, B: int,
                    alpha: Dict[str, Tuple[torch.Tensor, int]], splits: Dict[str, Tuple[torch.Tensor, int]],
                    G: torch.Tensor) -> Tuple[Dict[str, torch.Tensor], Dict[str, torch.Tensor]]:
    """Reverse pass of the lower bound of a DAG task (what autograd computes through
    crown_ibp.py:1669-2051 for alpha_beta_crown.py:913-923): dL/dalpha and dL/dbeta per
    ReLU ([B, n]), with G = dL/dlb per coefficient row.

    GA[v] = dL/dA_v for the backward state A_v of value v.  A_v is read once, by the
    backward of v's producer, so the ops run in forward order and each defines the
    gradient of its output from those of its inputs: the concretization seeds the input;
    linear GA[y] = GA[x] W^T + G bias^T; conv2d the forward convolution of GA[x] plus
    G bias^T; relu through the relaxation (bf_relu_grad, which also reduces dL/dalpha and
    dL/dbeta); add the sum of its operands' gradients (plus G c^T for a constant c);
    concat the concatenation of its operands' gradients; flatten/reshape the same rows."""
    task = _module_task(module)
    params = module.params
    dev = spec.center.device
    stream = _lib.stream_handle()
    S = int(saved["S"])
    M = B * S
    A_in = saved["input_A"]
    I = int(A_in.shape[1])
    center, rad, eps = _input_center_radius(spec, B, I)
    GA: Dict[str, torch.Tensor] = {}
    g0 = torch.empty(M, I, device=dev)
    with _timed("concretize_dense_grad", 0.0, 4.0 * 3 * M * I):
        _lib.call("bf_concretize_dense_grad", _lib.ptr(A_in), B, S, I, _lib.ptr(center), _lib.ptr(rad), eps,
                  input_norm_p(spec.perturbation), _lib.ptr(G), _lib.ptr(g0), stream)
    GA[spec.value_name] = g0
    g_alpha: Dict[str, torch.Tensor] = {}
    g_beta: Dict[str, torch.Tensor] = {}
    ran = saved["ran"]
    for op_index, op in enumerate(task.ops):
        if op_index not in ran:
            continue
        t = op.op_type
        y = op.outputs[0]
        x = op.inputs[0]
        if t == "linear":
            W = params[op.inputs[1]].contiguous()
            bias = params[op.inputs[2]].contiguous() if len(op.inputs) == 3 else None
            n_out, n_in = int(W.shape[0]), int(W.shape[1])
            gt = torch.empty(M, n_out, device=dev)
            wsz = int(_lib.load().bf_gemm_rank1_workspace(M, n_out, n_in))
            ws = torch.empty(wsz, device=dev) if wsz else None
            with _timed("grad_gemm", 2.0 * M * n_in * n_out, 4.0 * (M * n_in + M * n_out + n_in * n_out)):
                _lib.call("bf_gemm_rank1", _lib.ptr(GA[x]), n_in, _lib.ptr(W), n_in, 1, _lib.ptr(gt), n_out, M,
                          n_out, n_in, S, _lib.ptr(G if bias is not None else None), _lib.ptr(bias), 0, _lib.ptr(ws),
                          wsz, stream)
            GA[y] = gt
        elif t == "conv2d":
            W = params[op.inputs[1]].contiguous()
            in_shape = trace.shapes[x]
            (sh, sw), (ph, pw), out_shape = _conv_geometry(op, W, in_shape)
            Ci, Hi, Wi = in_shape
            Co, Ho, Wo = out_shape
            KH, KW = int(W.shape[2]), int(W.shape[3])
            vec = _conv_bias_map(params[op.inputs[2]], out_shape) if len(op.inputs) == 3 else None
            gt = torch.empty(M, Co * Ho * Wo, device=dev)
            with _timed("grad_conv", 2.0 * M * Co * Ho * Wo * Ci * KH * KW, 4.0 * (M * Ci * Hi * Wi + M * Co * Ho * Wo)):
                _lib.call("bf_conv2d_rows", _lib.ptr(GA[x]), 1, M, Ci, Hi, Wi, _lib.ptr(W), 0, Co, KH, KW, sh, sw, ph,
                          pw, Ho, Wo, _lib.ptr(gt), _lib.ptr(G if vec is not None else None), _lib.ptr(vec), 1, 0,
                          stream)
            GA[y] = gt
        elif t == "relu":
            pre = trace.relu_pre[x]
            n = _numel(pre.lower.shape[1:])
            a_t, a_ld = alpha.get(x, (None, 0))
            sp, sp_ld = splits.get(x, (None, 0))
            ga = torch.empty(B, n, device=dev)
            gb = torch.empty(B, n, device=dev)
            g_in = torch.empty(M, n, device=dev)
            with _timed("relu_grad", 0.0, 4.0 * (3 * M * n + 4 * B * n)):
                _lib.call("bf_relu_grad", _lib.ptr(GA[x]), _lib.ptr(saved["relu_A"][op_index]), S * n, B, S, n,
                          _lib.ptr(pre.lower.reshape(B, n)), _lib.ptr(pre.upper.reshape(B, n)), _lib.ptr(a_t), a_ld,
                          _lib.ptr(G), _lib.ptr(sp), sp_ld, _lib.ptr(g_in), _lib.ptr(ga), _lib.ptr(gb), stream)
            g_alpha[x] = ga
            g_beta[x] = gb
            GA[y] = g_in
        elif t in ("flatten", "reshape"):
            GA[y] = GA[x]
        elif t == "add":
            n = _numel(trace.shapes[y])
            acc = None
            for name in op.inputs:
                if name in trace.shapes:
                    if acc is None:
                        acc = GA[name]
                        continue
                    out = torch.empty(M, n, device=dev)
                    _lib.call("bf_rows_add", _lib.ptr(acc), _lib.ptr(GA[name]), M, n, S, None, None, 0, _lib.ptr(out),
                              stream)
                    acc = out
                else:
                    c = params[name].to(device=dev, dtype=torch.float32).reshape(B, n).contiguous()
                    out = torch.empty(M, n, device=dev)
                    _lib.call("bf_rows_add", _lib.ptr(acc), None, M, n, S, _lib.ptr(G), _lib.ptr(c), n, _lib.ptr(out),
                              stream)
                    acc = out
            GA[y] = acc
        elif t == "concat":
            parts = [GA[name].reshape(M, trace.shapes[name][0], -1) for name in op.inputs]
            GA[y] = torch.cat(parts, dim=1).reshape(M, -1)
    return g_alpha, g_beta


def run_crown_ibp_dag(
    module: BFTaskModule,
    input_spec,
    *,
    linear_spec_C: Optional[torch.Tensor] = None,
    output_value: Optional[str] = None,
    relu_alpha: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_add_coeff_l: Optional[Dict[str, torch.Tensor]] = None,
    relu_split_state: Optional[Dict[str, torch.Tensor]] = None,
) -> IntervalState:
    """run_crown_ibp_mlp (crown_ibp.py:2054-2133) on a DAG task."""
    spec = normalize_input_spec(input_spec)
    trace = forward_ibp_trace_dag(module, spec, relu_split_state=relu_split_state)
    return crown_backward_dag(module, spec, trace, linear_spec_C=linear_spec_C, output_value=output_value,
                              relu_alpha=relu_alpha, relu_pre_add_coeff_l=relu_pre_add_coeff_l)
