"""CPU restatement of the reference CROWN-IBP path (test infrastructure only).

Follows, op by op and with the same torch operations and association order:

* IBP forward trace -- boundflow/runtime/crown_ibp.py:101-342
* ReLU split application -- boundflow/runtime/crown_ibp.py:70-98
* Input-layer concretize_matmul -- boundflow/runtime/perturbation.py:102-173 (Lp ball),
  boundflow/runtime/perturbation.py:282-325 (box)
* Interval affine transformer -- boundflow/domains/interval.py:32-91
* Backward-state init -- boundflow/runtime/crown_ibp.py:672-719
* ReLU relaxation -- boundflow/runtime/crown_ibp.py:722-758, 1176-1208, 940-1070
* Dense ReLU backward -- boundflow/runtime/crown_ibp.py:1211-1298
* Linear / conv2d / flatten backward -- boundflow/runtime/crown_ibp.py:1073-1173
* Lazy coefficient operators (Dense, RightMatmul, ReshapeInput, Conv2d) --
  boundflow/runtime/linear_operator.py:299-720, 908-1092, 1378-1477
* Backward driver -- boundflow/runtime/crown_ibp.py:1669-2051, with the DAG pieces: fan-in
  accumulation (crown_ibp.py:874-937), add and concat adjoints (crown_ibp.py:1928-2030),
  AddLinearOperator / SliceInputLinearOperator (linear_operator.py:285-296, 1096-1340)
* concretize_affine -- boundflow/runtime/perturbation.py:175-222, 327-359
* Fused region reference -- boundflow/runtime/fused_crown.py:330-400
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, Mapping, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from boundflow_amd.ir import BFTaskModule
from boundflow_amd.spec import (
    BoxPerturbation,
    InputSpec,
    IntervalState,
    LpBallPerturbation,
    normalize_input_spec,
)


def _prod(shape: Sequence[int]) -> int:
    out = 1
    for d in shape:
        out *= int(d)
    return int(out)


def _pair(v: Any) -> Tuple[int, int]:
    if isinstance(v, int):
        return (int(v), int(v))
    if len(v) == 1:
        return (int(v[0]), int(v[0]))
    return (int(v[0]), int(v[1]))


# ---------------------------------------------------------------------------
# Input perturbation arithmetic (boundflow/runtime/perturbation.py)
# ---------------------------------------------------------------------------


def _input_marker(spec: InputSpec):
    return ("__input__", spec)


def _dual_row_norm(weight: torch.Tensor, p: str, dim: int) -> torch.Tensor:
    """Dual norm of each row over the Lp ball (perturbation.py:126-133): sum |w| for
    Linf, the L2 norm for L2, max |w| for L1."""
    if p == "inf":
        return weight.abs().sum(dim=dim)
    if p == "2":
        return torch.linalg.vector_norm(weight, ord=2, dim=dim)
    if p == "1":
        return weight.abs().amax(dim=dim)
    raise ValueError(f"unsupported p: {p!r}")


def concretize_matmul(spec: InputSpec, center: torch.Tensor, weight: torch.Tensor, bias):
    """perturbation.py:102-173 (Lp ball, p in {inf, 2, 1}) and :282-325 (box), rank-2 weights."""
    p = spec.perturbation
    if isinstance(p, LpBallPerturbation):
        eps = float(p.eps)
        out_center = center.matmul(weight.t())
        row_norm = _dual_row_norm(weight, p.normalized_p(), dim=1)
        deviation = eps * row_norm.unsqueeze(0)
        lb = out_center - deviation
        ub = out_center + deviation
        if bias is not None:
            lb = lb + bias
            ub = ub + bias
        return lb, ub
    midpoint = (p.lower + p.upper) / 2.0
    radius = (p.upper - p.lower) / 2.0
    output_center = midpoint.matmul(weight.t())
    deviation = radius.matmul(weight.abs().t())
    lower = output_center - deviation
    upper = output_center + deviation
    if bias is not None:
        lower = lower + bias
        upper = upper + bias
    return lower, upper


def interval_affine(l: torch.Tensor, u: torch.Tensor, w: torch.Tensor, b, attrs: Mapping[str, Any]):
    """domains/interval.py:32-86 (W+/W- form for linear and conv2d)."""
    if b is None:
        b = torch.as_tensor(0.0, device=l.device)
    op = attrs.get("op")
    if op == "conv2d":
        stride = _pair(attrs.get("stride", 1))
        padding = _pair(attrs.get("padding", 0))
        dilation = _pair(attrs.get("dilation", 1))
        groups = int(attrs.get("groups", 1))
        w_pos = torch.clamp(w, min=0.0)
        w_neg = torch.clamp(w, max=0.0)
        kw = dict(bias=None, stride=stride, padding=padding, dilation=dilation, groups=groups)
        y_l = F.conv2d(l, w_pos, **kw) + F.conv2d(u, w_neg, **kw)
        y_u = F.conv2d(u, w_pos, **kw) + F.conv2d(l, w_neg, **kw)
        y_l = y_l + b.view(1, -1, 1, 1) if b.dim() > 0 else y_l + b
        y_u = y_u + b.view(1, -1, 1, 1) if b.dim() > 0 else y_u + b
        return y_l, y_u
    w_pos = torch.clamp(w, min=0.0)
    w_neg = torch.clamp(w, max=0.0)
    y_l = l.matmul(w_pos.t()) + u.matmul(w_neg.t())
    y_u = u.matmul(w_pos.t()) + l.matmul(w_neg.t())
    return y_l + b, y_u + b


def broadcast_split(split: torch.Tensor, pre_lower: torch.Tensor) -> torch.Tensor:
    """relu_shape_utils.py:82-115: split int tensor -> [B, flat]."""
    logical = tuple(int(d) for d in pre_lower.shape[1:])
    flat = _prod(logical)
    batch = int(pre_lower.shape[0])
    if split.dim() == 0:
        return split.reshape(1, 1).expand(batch, flat)
    if tuple(split.shape) == logical or (split.dim() == 1 and int(split.shape[0]) == flat):
        return split.reshape(1, flat).expand(batch, flat)
    if int(split.shape[0]) == 1 and split.numel() == flat:
        return split.reshape(1, flat).expand(batch, flat)
    if int(split.shape[0]) == batch and split.numel() == batch * flat:
        return split.reshape(batch, flat)
    raise ValueError(f"split shape {tuple(split.shape)} cannot broadcast to {(batch, flat)}")


def apply_relu_split(pre: IntervalState, split: torch.Tensor, *, name: str) -> IntervalState:
    """crown_ibp.py:70-98."""
    split_b = broadcast_split(split, pre.lower)
    lower = pre.lower.reshape(int(pre.lower.shape[0]), -1)
    upper = pre.upper.reshape(int(pre.upper.shape[0]), -1)
    active = split_b > 0
    inactive = split_b < 0
    if not active.any() and not inactive.any():
        return pre
    if active.any():
        lower = torch.where(active, torch.maximum(lower, torch.zeros_like(lower)), lower)
    if inactive.any():
        upper = torch.where(inactive, torch.minimum(upper, torch.zeros_like(upper)), upper)
    if (lower > upper).any():
        raise ValueError(f"infeasible relu split for {name}: lower>upper after applying split")
    return IntervalState(lower=lower.reshape_as(pre.lower), upper=upper.reshape_as(pre.upper))


def concat_axis(axis_raw: Any, rank_with_batch: int) -> int:
    """dag_utils.py:6-20: the feature axis of [B, F] or the channel axis of [B, C, H, W]."""
    axis = int(axis_raw)
    if rank_with_batch == 2:
        if axis in (1, -1):
            return 1
        raise NotImplementedError(f"concat: only the feature axis of a rank-2 value, got axis={axis}")
    if rank_with_batch == 4:
        if axis in (1, -3):
            return 1
        raise NotImplementedError(f"concat: only the channel axis of a rank-4 value, got axis={axis}")
    raise NotImplementedError(f"concat: only rank-2 or rank-4 values, got rank={rank_with_batch}")


def check_concat_shapes(shapes: Sequence[Tuple[int, ...]], axis: int) -> int:
    """dag_utils.py:23-47: equal rank and equal non-axis dims; returns the concatenated axis size."""
    ref = tuple(int(d) for d in shapes[0])
    total = ref[axis]
    for shp in shapes[1:]:
        shp = tuple(int(d) for d in shp)
        if len(shp) != len(ref) or any(a != b for i, (a, b) in enumerate(zip(ref, shp)) if i != axis):
            raise NotImplementedError(f"concat: shapes {ref} and {shp} differ off the concat axis")
        total += shp[axis]
    return total


def forward_ibp_trace(
    module: BFTaskModule,
    spec: InputSpec,
    *,
    relu_split_state: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_constraints: Optional[Mapping[str, IntervalState]] = None,
) -> Tuple[Dict[str, IntervalState], Dict[str, IntervalState]]:
    """crown_ibp.py:101-342 for linear/conv2d/relu/add/concat/flatten/reshape."""
    task = module.get_entry_task()
    params = module.params
    env: Dict[str, Any] = {spec.value_name: _input_marker(spec)}
    interval_env: Dict[str, IntervalState] = {}
    relu_pre: Dict[str, IntervalState] = {}

    def is_input(s):
        return isinstance(s, tuple) and s and s[0] == "__input__"

    def ensure_interval(s) -> IntervalState:
        if isinstance(s, IntervalState):
            return s
        sp: InputSpec = s[1]
        lb, ub = sp.perturbation.bounding_box(sp.center)
        return IntervalState(lower=lb, upper=ub)

    def get_state(name):
        if name in env:
            return env[name]
        t = params[name]
        return IntervalState(lower=t, upper=t)

    for op in task.ops:
        t = op.op_type
        if t == "linear":
            xs = get_state(op.inputs[0])
            w = params[op.inputs[1]]
            b = params[op.inputs[2]] if len(op.inputs) == 3 else None
            if is_input(xs):
                lb, ub = concretize_matmul(xs[1], xs[1].center, w, b)
            else:
                x = ensure_interval(xs)
                lb, ub = interval_affine(x.lower, x.upper, w, b, {"op": "linear"})
            y = IntervalState(lb, ub)
        elif t == "conv2d":
            x = ensure_interval(get_state(op.inputs[0]))
            w = params[op.inputs[1]]
            b = params[op.inputs[2]] if len(op.inputs) == 3 else None
            attrs = dict(op.attrs)
            attrs.setdefault("op", "conv2d")
            lb, ub = interval_affine(x.lower, x.upper, w, b, attrs)
            y = IntervalState(lb, ub)
        elif t == "relu":
            name = op.inputs[0]
            x = ensure_interval(get_state(name))
            if relu_pre_constraints is not None:
                c = relu_pre_constraints[name]
                lower = torch.maximum(x.lower, c.lower)
                upper = torch.minimum(x.upper, c.upper)
                if bool((lower > upper).any().item()):
                    raise ValueError(f"infeasible ReLU pre-activation intersection for {name}")
                x = IntervalState(lower, upper)
            if relu_split_state is not None and name in relu_split_state:
                x = apply_relu_split(x, relu_split_state[name], name=name)
            relu_pre[name] = x
            y = IntervalState(torch.relu(x.lower), torch.relu(x.upper))
        elif t == "add":
            a = ensure_interval(get_state(op.inputs[0]))
            b2 = ensure_interval(get_state(op.inputs[1]))
            if tuple(a.lower.shape) != tuple(b2.lower.shape):
                raise NotImplementedError(
                    "_forward_ibp_trace_mlp only supports add with exact same-shape inputs; "
                    f"got {tuple(a.lower.shape)} and {tuple(b2.lower.shape)}")
            y = IntervalState(a.lower + b2.lower, a.upper + b2.upper)
        elif t == "concat":
            # crown_ibp.py:235-257 with dag_utils.py:6-47
            if len(op.inputs) < 2:
                raise ValueError(f"concat expects at least 2 inputs, got {len(op.inputs)}")
            parts = [ensure_interval(get_state(name)) for name in op.inputs]
            axis = concat_axis(op.attrs.get("axis", 1), int(parts[0].lower.dim()))
            check_concat_shapes([tuple(p.lower.shape) for p in parts], axis)
            y = IntervalState(torch.cat([p.lower for p in parts], dim=axis),
                              torch.cat([p.upper for p in parts], dim=axis))
        elif t in ("flatten", "reshape"):
            xs = get_state(op.inputs[0])
            if is_input(xs):
                sp: InputSpec = xs[1]
                if t == "flatten":
                    f = lambda z: torch.flatten(z, start_dim=1, end_dim=-1)  # noqa: E731
                else:
                    shape = tuple(int(d) for d in op.attrs["shape"])
                    f = lambda z: z.reshape(shape)  # noqa: E731
                pert = sp.perturbation
                if isinstance(pert, BoxPerturbation):
                    pert = BoxPerturbation(lower=f(pert.lower), upper=f(pert.upper))
                new_spec = InputSpec(value_name=sp.value_name, center=f(sp.center), perturbation=pert)
                env[op.outputs[0]] = _input_marker(new_spec)
                if isinstance(pert, BoxPerturbation):
                    interval_env[op.outputs[0]] = IntervalState(pert.lower, pert.upper)
                continue
            x = ensure_interval(xs)
            if t == "flatten":
                y = IntervalState(torch.flatten(x.lower, 1, -1), torch.flatten(x.upper, 1, -1))
            else:
                shape = tuple(int(d) for d in op.attrs["shape"])
                y = IntervalState(x.lower.reshape(shape), x.upper.reshape(shape))
        else:
            raise NotImplementedError(f"oracle forward: unsupported op_type {t}")
        env[op.outputs[0]] = y
        interval_env[op.outputs[0]] = y
    return interval_env, relu_pre


# ---------------------------------------------------------------------------
# Lazy coefficient operators (boundflow/runtime/linear_operator.py)
# ---------------------------------------------------------------------------


def _flatten_contract_input(vec: torch.Tensor, batch: int, input_shape: Tuple[int, ...]) -> torch.Tensor:
    """linear_operator.py:77-108."""
    flat = _prod(input_shape)
    if tuple(vec.shape) == tuple(input_shape):
        return vec.reshape(1, flat).expand(batch, -1)
    if tuple(vec.shape) == (batch,) + tuple(input_shape):
        return vec.reshape(batch, flat)
    if len(input_shape) == 1 and vec.dim() == 1 and int(vec.shape[0]) == flat:
        return vec.reshape(1, flat).expand(batch, -1)
    if len(input_shape) == 1 and vec.dim() == 2 and tuple(vec.shape) == (batch, flat):
        return vec
    raise ValueError(f"contract vec shape mismatch: {tuple(vec.shape)} vs {input_shape}")


class DenseOp:
    """linear_operator.py:299-456."""

    def __init__(self, coeffs: torch.Tensor, input_shape: Tuple[int, ...]):
        self.coeffs = coeffs
        self.input_shape = tuple(int(d) for d in input_shape)

    @property
    def shape(self):
        c = self.coeffs
        return (int(c.shape[0]), int(c.shape[1]), _prod(self.input_shape))

    @property
    def spec_dim(self):
        return self.shape[1]

    def flat(self):
        return self.coeffs.reshape(self.shape)

    def center_term(self, center):
        return torch.einsum("bki,bi->bk", self.flat(), center.reshape(self.shape[0], -1))

    def row_abs_sum(self):
        return self.flat().abs().sum(dim=2)

    def contract_input(self, vec):
        return torch.einsum("bki,bi->bk", self.flat(), _flatten_contract_input(vec, self.shape[0], self.input_shape))

    def to_dense(self):
        return self.flat()

    def feature_rows(self, shape):
        return self.coeffs.reshape(self.shape[0] * self.spec_dim, *shape)


class RightMatmulOp:
    """linear_operator.py:459-586 (lazy A @ rhs)."""

    def __init__(self, base, rhs: torch.Tensor):
        self.base = base
        self.rhs = rhs
        self.input_shape = (int(rhs.shape[1]),)

    @property
    def shape(self):
        return (self.base.shape[0], self.base.shape[1], int(self.rhs.shape[1]))

    @property
    def spec_dim(self):
        return self.base.spec_dim

    def center_term(self, center):
        flat = center.reshape(self.shape[0], -1)
        return self.base.center_term(flat.matmul(self.rhs.t()))

    def row_abs_sum(self):
        return self.to_dense().abs().sum(dim=2)

    def contract_input(self, vec):
        flat = _flatten_contract_input(vec, self.shape[0], self.input_shape)
        return self.base.contract_input(flat.matmul(self.rhs.t()))

    def to_dense(self):
        return torch.einsum("bko,oi->bki", self.base.to_dense(), self.rhs)

    def feature_rows(self, shape):
        return self.to_dense().reshape(self.shape[0] * self.spec_dim, *shape)


class ReshapeOp:
    """linear_operator.py:588-720."""

    def __init__(self, base, input_shape):
        self.base = base
        self.input_shape = tuple(int(d) for d in input_shape)

    @property
    def shape(self):
        return self.base.shape

    @property
    def spec_dim(self):
        return self.base.spec_dim

    def _for_base(self, flat):
        return flat.view(int(flat.shape[0]), *self.base.input_shape)

    def center_term(self, center):
        return self.base.center_term(self._for_base(center.reshape(self.shape[0], -1)))

    def row_abs_sum(self):
        return self.base.row_abs_sum()

    def contract_input(self, vec):
        flat = _flatten_contract_input(vec, self.shape[0], self.input_shape)
        return self.base.contract_input(self._for_base(flat))

    def to_dense(self):
        return self.base.to_dense()

    def feature_rows(self, shape):
        if len(self.base.input_shape) == 3:
            return self.base.feature_rows(self.base.input_shape).reshape(self.shape[0] * self.spec_dim, *shape)
        return self.base.to_dense().reshape(self.shape[0] * self.spec_dim, *shape)


def conv_output_padding(input_shape, output_shape, weight, stride, padding, dilation):
    """linear_operator.py:140-163."""
    kh, kw = int(weight.shape[2]), int(weight.shape[3])
    oph = int(input_shape[1]) - ((int(output_shape[1]) - 1) * stride[0] - 2 * padding[0] + dilation[0] * (kh - 1) + 1)
    opw = int(input_shape[2]) - ((int(output_shape[2]) - 1) * stride[1] - 2 * padding[1] + dilation[1] * (kw - 1) + 1)
    return (oph, opw)


class Conv2dOp:
    """linear_operator.py:908-1092 (lazy A @ Conv2d)."""

    def __init__(self, base, weight, stride, padding, dilation, groups, input_shape):
        self.base = base
        self.weight = weight
        self.stride = stride
        self.padding = padding
        self.dilation = dilation
        self.groups = groups
        self.input_shape = tuple(int(d) for d in input_shape)

    @property
    def shape(self):
        return (self.base.shape[0], self.base.shape[1], _prod(self.input_shape))

    @property
    def spec_dim(self):
        return self.base.spec_dim

    def _conv(self, flat):
        x = flat.view(int(flat.shape[0]), *self.input_shape)
        return F.conv2d(x, self.weight, bias=None, stride=self.stride, padding=self.padding,
                        dilation=self.dilation, groups=self.groups)

    def center_term(self, center):
        return self.base.center_term(self._conv(center.reshape(self.shape[0], -1)))

    def contract_input(self, vec):
        flat = _flatten_contract_input(vec, self.shape[0], self.input_shape)
        return self.base.contract_input(self._conv(flat))

    def _transpose(self, base_rows):
        out_shape = tuple(int(d) for d in self.base.input_shape)
        opad = conv_output_padding(self.input_shape, out_shape, self.weight, self.stride, self.padding, self.dilation)
        return F.conv_transpose2d(base_rows, self.weight, bias=None, stride=self.stride, padding=self.padding,
                                  output_padding=opad, dilation=self.dilation, groups=self.groups)

    def feature_rows(self, shape):
        base_rows = self.base.feature_rows(tuple(int(d) for d in self.base.input_shape))
        return self._transpose(base_rows).reshape(self.shape[0] * self.spec_dim, *shape)

    def row_abs_sum(self):
        rows = self.feature_rows(self.input_shape)
        return rows.abs().sum(dim=(1, 2, 3)).view(self.shape[0], self.spec_dim)

    def to_dense(self):
        out_shape = tuple(int(d) for d in self.base.input_shape)
        base_dense = self.base.to_dense().view(self.shape[0] * self.spec_dim, *out_shape)
        return self._transpose(base_dense).view(self.shape[0], self.spec_dim, -1)


class AddOp:
    """linear_operator.py:1096-1235 (lazy sum of two operators of one input shape)."""

    def __init__(self, lhs, rhs):
        if tuple(lhs.shape) != tuple(rhs.shape) or tuple(lhs.input_shape) != tuple(rhs.input_shape):
            raise ValueError(f"add shape mismatch: {lhs.shape}/{lhs.input_shape} vs {rhs.shape}/{rhs.input_shape}")
        self.lhs = lhs
        self.rhs = rhs
        self.input_shape = tuple(lhs.input_shape)

    @property
    def shape(self):
        return self.lhs.shape

    @property
    def spec_dim(self):
        return self.lhs.spec_dim

    def center_term(self, center):
        return self.lhs.center_term(center) + self.rhs.center_term(center)

    def contract_input(self, vec):
        return self.lhs.contract_input(vec) + self.rhs.contract_input(vec)

    def row_abs_sum(self):
        return self.to_dense().abs().sum(dim=2)

    def to_dense(self):
        return self.lhs.to_dense() + self.rhs.to_dense()

    def feature_rows(self, shape):
        return self.to_dense().reshape(self.shape[0] * self.spec_dim, *shape)


class SliceOp:
    """linear_operator.py:1237-1340: the columns [start, stop) of the leading per-sample axis
    (features of [F], channels of [C, H, W]) of the base operator's input."""

    def __init__(self, base, input_shape, start: int, stop: int):
        self.base = base
        self.input_shape = tuple(int(d) for d in input_shape)
        self.start = int(start)
        self.stop = int(stop)
        base_shape = tuple(int(d) for d in base.input_shape)
        if len(base_shape) != len(self.input_shape) or self.stop - self.start != self.input_shape[0] \
                or base_shape[1:] != self.input_shape[1:] or not 0 <= self.start <= self.stop <= base_shape[0]:
            raise ValueError(f"slice_input mismatch: base {base_shape}, slice {self.input_shape} "
                             f"[{self.start}:{self.stop}]")

    @property
    def shape(self):
        return (self.base.shape[0], self.base.shape[1], _prod(self.input_shape))

    @property
    def spec_dim(self):
        return self.base.spec_dim

    def _embed(self, flat):
        """A [B, prod(input_shape)] vector placed, zero-padded, in the base input."""
        b = int(flat.shape[0])
        full = torch.zeros((b,) + tuple(self.base.input_shape), dtype=flat.dtype, device=flat.device)
        full[:, self.start:self.stop] = flat.reshape((b,) + self.input_shape)
        return full

    def center_term(self, center):
        return self.base.center_term(self._embed(center.reshape(self.shape[0], -1)))

    def contract_input(self, vec):
        return self.base.contract_input(self._embed(_flatten_contract_input(vec, self.shape[0], self.input_shape)))

    def row_abs_sum(self):
        return self.to_dense().abs().sum(dim=2)

    def to_dense(self):
        b, k = self.shape[0], self.spec_dim
        dense = self.base.to_dense().reshape((b, k) + tuple(self.base.input_shape))
        return dense[:, :, self.start:self.stop].reshape(b, k, -1)

    def feature_rows(self, shape):
        return self.to_dense().reshape(self.shape[0] * self.spec_dim, *shape)


def reshape_input(op, shape):
    shape = tuple(int(d) for d in shape)
    if tuple(op.input_shape) == shape:
        return op
    if isinstance(op, ReshapeOp):
        return ReshapeOp(op.base, shape)
    return ReshapeOp(op, shape)


def conv2d_right(op, weight, stride, padding, dilation, groups, input_shape, output_shape):
    op = reshape_input(op, output_shape)
    return Conv2dOp(op, weight, stride, padding, dilation, groups, input_shape)


def matmul_right(op, rhs):
    if isinstance(op, RightMatmulOp):
        return RightMatmulOp(op.base, op.rhs.matmul(rhs))
    return RightMatmulOp(op, rhs)


# ---------------------------------------------------------------------------
# ReLU relaxation and dense backward (boundflow/runtime/crown_ibp.py)
# ---------------------------------------------------------------------------


def relu_relax(l: torch.Tensor, u: torch.Tensor):
    """crown_ibp.py:722-758 (upper chord, ZERO lower slope)."""
    pos = l >= 0
    neg = u <= 0
    amb = (~pos) & (~neg)
    alpha_u = torch.empty_like(l)
    beta_u = torch.empty_like(l)
    alpha_l = torch.empty_like(l)
    beta_l = torch.empty_like(l)
    alpha_u[pos] = 1.0
    beta_u[pos] = 0.0
    alpha_l[pos] = 1.0
    beta_l[pos] = 0.0
    alpha_u[neg] = 0.0
    beta_u[neg] = 0.0
    alpha_l[neg] = 0.0
    beta_l[neg] = 0.0
    if amb.any():
        l_amb = l[amb]
        u_amb = u[amb]
        denom = (u_amb - l_amb).clamp_min(torch.finfo(l.dtype).eps)
        a = u_amb / denom
        alpha_u[amb] = a
        beta_u[amb] = -l_amb * a
        alpha_l[amb] = 0.0
        beta_l[amb] = 0.0
    return alpha_u, beta_u, alpha_l, beta_l


def broadcast_alpha(alpha: torch.Tensor, pre: IntervalState) -> torch.Tensor:
    """crown_ibp.py:940-1001 (shape rules) ending in clamp(0,1)."""
    logical = tuple(int(d) for d in pre.lower.shape[1:])
    flat = _prod(logical)
    batch = int(pre.lower.shape[0])
    if alpha.dim() == 0:
        out = alpha.reshape(1, 1).expand(batch, flat)
    elif tuple(alpha.shape) == logical or (alpha.dim() == 1 and int(alpha.shape[0]) == flat):
        out = alpha.reshape(1, flat).expand(batch, flat)
    elif int(alpha.shape[0]) == 1 and alpha.numel() == flat:
        out = alpha.reshape(1, flat).expand(batch, flat)
    elif int(alpha.shape[0]) == batch and alpha.numel() == batch * flat:
        out = alpha.reshape(batch, flat)
    else:
        raise ValueError(f"alpha shape {tuple(alpha.shape)} cannot broadcast to {(batch, flat)}")
    return out.clamp(0.0, 1.0)


def broadcast_pre_add(add: torch.Tensor, batch: int, flat: int) -> torch.Tensor:
    """crown_ibp.py:1004-1052."""
    if add.dim() == 0:
        add = add.expand(flat)
    if add.dim() == 1:
        return add.view(1, -1).expand(batch, -1)
    if add.dim() == 2:
        return add.expand(batch, -1) if int(add.shape[0]) == 1 else add
    if add.numel() == flat:
        return add.reshape(1, flat).expand(batch, -1)
    return add.reshape(batch, flat)


def relu_backward_relaxation(pre: IntervalState, name: str, relu_alpha):
    """crown_ibp.py:1176-1208."""
    l = pre.lower.reshape(int(pre.lower.shape[0]), -1)
    u = pre.upper.reshape(int(pre.upper.shape[0]), -1)
    alpha_u, beta_u, alpha_l, beta_l = relu_relax(l, u)
    if relu_alpha is not None and name in relu_alpha:
        a = broadcast_alpha(relu_alpha[name], pre)
        amb = (l < 0) & (u > 0)
        if amb.any():
            alpha_l = torch.where(amb, a, alpha_l)
    return (l, u), alpha_u, beta_u, alpha_l, beta_l


def relu_backward_dense(A_u, A_l, b_u, b_l, *, pre, name, relu_alpha=None, add_u=None, add_l=None):
    """crown_ibp.py:1211-1298 (dense reference equations)."""
    _pf, alpha_u, beta_u, alpha_l, beta_l = relu_backward_relaxation(pre, name, relu_alpha)
    sel_alpha_u = torch.where(A_u >= 0, alpha_u.unsqueeze(1), alpha_l.unsqueeze(1))
    sel_beta_u = torch.where(A_u >= 0, beta_u.unsqueeze(1), beta_l.unsqueeze(1))
    out_b_u = b_u + (A_u * sel_beta_u).sum(dim=2)
    out_A_u = A_u * sel_alpha_u
    if add_u is not None and name in add_u:
        out_A_u = out_A_u + broadcast_pre_add(add_u[name], int(A_u.shape[0]), int(A_u.shape[2])).unsqueeze(1)
    sel_alpha_l = torch.where(A_l >= 0, alpha_l.unsqueeze(1), alpha_u.unsqueeze(1))
    sel_beta_l = torch.where(A_l >= 0, beta_l.unsqueeze(1), beta_u.unsqueeze(1))
    out_b_l = b_l + (A_l * sel_beta_l).sum(dim=2)
    out_A_l = A_l * sel_alpha_l
    if add_l is not None and name in add_l:
        out_A_l = out_A_l + broadcast_pre_add(add_l[name], int(A_l.shape[0]), int(A_l.shape[2])).unsqueeze(1)
    return out_A_u, out_A_l, out_b_u, out_b_l


@dataclass
class _State:
    A_u: Any
    A_l: Any
    b_u: torch.Tensor
    b_l: torch.Tensor


def _value_shape(spec: InputSpec, interval_env, name) -> Tuple[int, ...]:
    if name == spec.value_name:
        return tuple(int(d) for d in spec.center.shape[1:])
    return tuple(int(d) for d in interval_env[name].lower.shape[1:])


def concretize_affine(spec: InputSpec, center: torch.Tensor, op, b):
    """perturbation.py:175-222 (Lp ball, p in {inf, 2, 1}) and :327-359 (box)."""
    p = spec.perturbation
    if isinstance(p, LpBallPerturbation):
        eps = float(p.eps)
        out_center = op.center_term(center)
        q = p.normalized_p()
        # row_l2_norm / row_abs_max of every reference operator reduce its dense
        # materialization (linear_operator.py:368-372, 518-522, 813-821, 991-997)
        row_norm = op.row_abs_sum() if q == "inf" else _dual_row_norm(op.to_dense(), q, dim=2)
        deviation = eps * row_norm
        return out_center - deviation + b, out_center + deviation + b
    midpoint = (p.lower + p.upper) / 2.0
    radius = (p.upper - p.lower) / 2.0
    output_center = op.center_term(midpoint)
    dense = op.to_dense()
    deviation = (dense.abs() * radius.reshape(int(center.shape[0]), 1, -1)).sum(dim=2)
    return output_center - deviation + b, output_center + deviation + b


def crown_backward_from_trace(
    module: BFTaskModule,
    spec: InputSpec,
    *,
    interval_env: Dict[str, IntervalState],
    relu_pre: Dict[str, IntervalState],
    linear_spec_C: Optional[torch.Tensor] = None,
    output_value: Optional[str] = None,
    relu_alpha: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_add_coeff_u: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_add_coeff_l: Optional[Dict[str, torch.Tensor]] = None,
    relu_influence_out: Optional[Dict[str, torch.Tensor]] = None,
) -> IntervalState:
    """crown_ibp.py:1669-2051: ops in reverse order, each popping the backward state of its
    output; a value read by several ops accumulates their contributions (crown_ibp.py:892-909)
    before its own op runs."""
    task = module.get_entry_task()
    params = module.params
    if output_value is None:
        output_value = task.output_values[0]
    y_out = interval_env[output_value]
    batch = int(y_out.lower.shape[0])
    output_shape = tuple(int(d) for d in y_out.lower.shape[1:])
    out_dim = _prod(output_shape)
    dtype = y_out.lower.dtype
    device = y_out.lower.device
    # _init_backward_state (crown_ibp.py:672-719)
    if linear_spec_C is None:
        A = torch.eye(out_dim, device=device, dtype=dtype).unsqueeze(0).expand(batch, out_dim, out_dim).clone()
        b0 = torch.zeros(batch, out_dim, device=device, dtype=dtype)
    else:
        C = linear_spec_C.to(device=device, dtype=dtype)
        if C.dim() == 2:
            C = C.unsqueeze(0).expand(batch, int(C.shape[0]), out_dim).clone()
        A = C
        b0 = torch.zeros(int(C.shape[0]), int(C.shape[1]), device=device, dtype=dtype)
    adjoints: Dict[str, _State] = {
        output_value: _State(DenseOp(A, output_shape), DenseOp(A.clone(), output_shape), b0, b0.clone())
    }
    # crown_ibp.py:912-919: values that depend on the input; other add operands are constants
    dynamic = set(interval_env.keys()) | {spec.value_name}

    def operand_box(name) -> IntervalState:
        if name == spec.value_name:
            lb, ub = spec.perturbation.bounding_box(spec.center)
            return IntervalState(lb, ub)
        if name in interval_env:
            return interval_env[name]
        t_ = params[name]
        return IntervalState(t_, t_)

    def accumulate(name, new: _State) -> None:
        shape = _value_shape(spec, interval_env, name)
        new = _State(reshape_input(new.A_u, shape), reshape_input(new.A_l, shape), new.b_u, new.b_l)
        cur = adjoints.get(name)
        if cur is not None:
            cur = _State(reshape_input(cur.A_u, shape), reshape_input(cur.A_l, shape), cur.b_u, cur.b_l)
            new = _State(AddOp(cur.A_u, new.A_u), AddOp(cur.A_l, new.A_l), cur.b_u + new.b_u, cur.b_l + new.b_l)
        adjoints[name] = new

    for op in reversed(task.ops):
        out_name = op.outputs[0]
        st = adjoints.pop(out_name, None)
        if st is None:
            continue
        t = op.op_type
        if t == "linear":
            w = params[op.inputs[1]]
            bias = params[op.inputs[2]] if len(op.inputs) == 3 else torch.zeros(int(w.shape[0]), dtype=dtype)
            new = _State(
                matmul_right(st.A_u, w),
                matmul_right(st.A_l, w),
                st.b_u + st.A_u.contract_input(bias),
                st.b_l + st.A_l.contract_input(bias),
            )
            in_name = op.inputs[0]
        elif t in ("flatten", "reshape"):
            in_name = op.inputs[0]
            shape = _value_shape(spec, interval_env, in_name)
            new = _State(reshape_input(st.A_u, shape), reshape_input(st.A_l, shape), st.b_u, st.b_l)
        elif t == "relu":
            name = op.inputs[0]
            pre = relu_pre[name]
            in_shape = tuple(int(d) for d in pre.lower.shape[1:])
            if relu_influence_out is not None:
                # crown_ibp.py:1810-1833: max over specs of the coefficient magnitudes at the ReLU
                if name in relu_influence_out:
                    raise ValueError(f"duplicate ReLU objective influence identity: {name}")
                cu = st.A_u.to_dense().reshape(batch, -1, *in_shape)
                cl = st.A_l.to_dense().reshape(batch, -1, *in_shape)
                relu_influence_out[name] = torch.maximum(cu.abs().amax(dim=1), cl.abs().amax(dim=1)).detach()
            if pre.lower.dim() != 2 and relu_pre_add_coeff_u is not None and name in relu_pre_add_coeff_u:
                # crown_ibp.py:1256-1260
                raise NotImplementedError(
                    f"run_crown_ibp_mlp only supports relu_pre_add_coeff_u on rank-2 pre-activations; got "
                    f"{tuple(pre.lower.shape)} for {name}")
            dA_u, dA_l, b_u, b_l = relu_backward_dense(
                st.A_u.to_dense(), st.A_l.to_dense(), st.b_u, st.b_l, pre=pre, name=name,
                relu_alpha=relu_alpha, add_u=relu_pre_add_coeff_u, add_l=relu_pre_add_coeff_l,
            )
            new = _State(DenseOp(dA_u, in_shape), DenseOp(dA_l, in_shape), b_u, b_l)
            in_name = name
        elif t == "conv2d":
            in_name = op.inputs[0]
            in_shape = _value_shape(spec, interval_env, in_name)
            out_shape = _value_shape(spec, interval_env, out_name)
            w = params[op.inputs[1]]
            bias = params[op.inputs[2]] if len(op.inputs) == 3 else None
            stride = _pair(op.attrs.get("stride", 1))
            padding = _pair(op.attrs.get("padding", 0))
            dilation = _pair(op.attrs.get("dilation", 1))
            groups = int(op.attrs.get("groups", 1))
            A_u = reshape_input(st.A_u, out_shape)
            A_l = reshape_input(st.A_l, out_shape)
            b_u, b_l = st.b_u, st.b_l
            if bias is not None:
                bias_map = bias.view(-1, 1, 1).expand(out_shape)
                b_u = b_u + A_u.contract_input(bias_map)
                b_l = b_l + A_l.contract_input(bias_map)
            new = _State(
                conv2d_right(A_u, w, stride, padding, dilation, groups, in_shape, out_shape),
                conv2d_right(A_l, w, stride, padding, dilation, groups, in_shape, out_shape),
                b_u, b_l,
            )
        elif t == "add":
            # crown_ibp.py:1928-1970: every dynamic operand receives the same coefficient; a
            # constant operand's contribution goes into the bias, which the first dynamic
            # operand carries (the others get zeros, crown_ibp.py:922-937)
            out_shape = _value_shape(spec, interval_env, out_name)
            A_u, A_l = reshape_input(st.A_u, out_shape), reshape_input(st.A_l, out_shape)
            cb_u, cb_l = st.b_u, st.b_l
            dyn = []
            for name in op.inputs:
                val = operand_box(name)
                if tuple(int(d) for d in val.lower.shape[1:]) != tuple(out_shape):
                    raise NotImplementedError(
                        f"add backward: only exact same-shape non-broadcast inputs; got output_shape={out_shape} "
                        f"input_shape={tuple(int(d) for d in val.lower.shape[1:])}")
                if name in dynamic:
                    dyn.append(name)
                else:
                    cb_u = cb_u + A_u.contract_input(val.lower)
                    cb_l = cb_l + A_l.contract_input(val.lower)
            for idx, name in enumerate(dyn):
                bu, bl = (cb_u, cb_l) if idx == 0 else (torch.zeros_like(cb_u), torch.zeros_like(cb_l))
                accumulate(name, _State(A_u, A_l, bu, bl))
            continue
        elif t == "concat":
            # crown_ibp.py:1972-2030: each operand receives its slice of the coefficient's
            # leading per-sample axis; the bias goes with the first operand
            out_shape = _value_shape(spec, interval_env, out_name)
            concat_axis(op.attrs.get("axis", 1), len(out_shape) + 1)
            A_u, A_l = reshape_input(st.A_u, out_shape), reshape_input(st.A_l, out_shape)
            shapes = [_value_shape(spec, interval_env, name) for name in op.inputs]
            total = check_concat_shapes(shapes, 0)
            start = 0
            for idx, (name, shp) in enumerate(zip(op.inputs, shapes)):
                if name not in dynamic:
                    raise NotImplementedError(f"concat backward: only dynamic tensor values, got {name}")
                stop = start + int(shp[0])
                bu, bl = (st.b_u, st.b_l) if idx == 0 else (torch.zeros_like(st.b_u), torch.zeros_like(st.b_l))
                accumulate(name, _State(SliceOp(A_u, shp, start, stop), SliceOp(A_l, shp, start, stop), bu, bl))
                start = stop
            if start != total or total != int(out_shape[0]):
                raise ValueError(f"concat backward shape mismatch: sliced={start} total={total} out={out_shape}")
            continue
        else:
            raise NotImplementedError(f"oracle backward: unsupported op_type {t}")
        accumulate(in_name, new)

    st = adjoints[spec.value_name]
    center_shape = tuple(int(d) for d in spec.center.shape[1:])
    A_u = reshape_input(st.A_u, center_shape)
    A_l = reshape_input(st.A_l, center_shape)
    _lb_u, ub_u = concretize_affine(spec, spec.center, A_u, st.b_u)
    lb_l, _ub_l = concretize_affine(spec, spec.center, A_l, st.b_l)
    return IntervalState(lower=lb_l, upper=ub_u)


def run_crown_ibp(
    module: BFTaskModule,
    input_spec,
    *,
    linear_spec_C: Optional[torch.Tensor] = None,
    output_value: Optional[str] = None,
    relu_alpha=None,
    relu_pre_add_coeff_u=None,
    relu_pre_add_coeff_l=None,
    relu_split_state=None,
) -> IntervalState:
    """crown_ibp.py:2054-2133 (run_crown_ibp_mlp)."""
    module.validate()
    spec = normalize_input_spec(input_spec)
    interval_env, relu_pre = forward_ibp_trace(module, spec, relu_split_state=relu_split_state)
    return crown_backward_from_trace(
        module, spec, interval_env=interval_env, relu_pre=relu_pre, linear_spec_C=linear_spec_C,
        output_value=output_value, relu_alpha=relu_alpha,
        relu_pre_add_coeff_u=relu_pre_add_coeff_u, relu_pre_add_coeff_l=relu_pre_add_coeff_l,
    )


def run_crown_all_intermediate(
    module: BFTaskModule,
    input_spec,
    *,
    linear_spec_C: torch.Tensor,
) -> Tuple[IntervalState, Dict[str, IntervalState]]:
    """CROWN with every intermediate pre-activation bound computed by CROWN.

    The reference has no single function for this; it is the layer-by-layer
    composition of the selected-neuron pattern
    (boundflow/runtime/native_intermediate_refinement.py:923-988): for each ReLU
    input in op order (after the first, whose IBP bound is already exact for a
    linear input layer), run CROWN with ``output_value`` = that pre-activation and
    ``C = I``, using the ReLU bounds refined so far, then intersect with the
    current bounds.  The final spec bound uses the refined bounds.
    """
    module.validate()
    spec = normalize_input_spec(input_spec)
    interval_env, relu_pre = forward_ibp_trace(module, spec)
    names = list(relu_pre.keys())
    for name in names[1:]:
        numel = int(relu_pre[name].lower[0].numel())
        eye = torch.eye(numel, dtype=relu_pre[name].lower.dtype)
        b = crown_backward_from_trace(module, spec, interval_env=interval_env, relu_pre=relu_pre,
                                      linear_spec_C=eye, output_value=name)
        cur = relu_pre[name]
        lower = torch.maximum(cur.lower.reshape(b.lower.shape), b.lower).reshape(cur.lower.shape)
        upper = torch.minimum(cur.upper.reshape(b.upper.shape), b.upper).reshape(cur.upper.shape)
        if bool((lower > upper).any()):
            raise ValueError("intermediate refinement intersection is infeasible")
        relu_pre[name] = IntervalState(lower, upper)
    final = crown_backward_from_trace(module, spec, interval_env=interval_env, relu_pre=relu_pre,
                                      linear_spec_C=linear_spec_C)
    return final, relu_pre


def fused_relu_affine_reference(A_u, A_l, alpha_u, alpha_l, beta_u, beta_l, weight, bias,
                                kind="linear", input_shape=None, output_shape=None, attrs=None):
    """fused_crown.py:330-400 (TorchDenseFusedCrownReference.run)."""
    A_u = A_u.reshape(A_u.shape[0], A_u.shape[1], -1)
    A_l = A_l.reshape(A_l.shape[0], A_l.shape[1], -1)
    scaled_u = torch.where(A_u >= 0, A_u * alpha_u[:, None], A_u * alpha_l[:, None])
    scaled_l = torch.where(A_l >= 0, A_l * alpha_l[:, None], A_l * alpha_u[:, None])
    delta_u = torch.where(A_u >= 0, A_u * beta_u[:, None], A_u * beta_l[:, None]).sum(2)
    delta_l = torch.where(A_l >= 0, A_l * beta_l[:, None], A_l * beta_u[:, None]).sum(2)
    if kind == "linear":
        if bias is not None:
            delta_u = delta_u + (scaled_u * bias).sum(2)
            delta_l = delta_l + (scaled_l * bias).sum(2)
        return scaled_u @ weight, scaled_l @ weight, delta_u, delta_l
    attrs = dict(attrs or {})
    stride = _pair(attrs.get("stride", 1))
    padding = _pair(attrs.get("padding", 0))
    dilation = _pair(attrs.get("dilation", 1))
    groups = int(attrs.get("groups", 1))
    opad = _pair(attrs.get("output_padding", 0))
    D, S = int(A_u.shape[0]), int(A_u.shape[1])
    prev = []
    for scaled in (scaled_u, scaled_l):
        prev.append(F.conv_transpose2d(scaled.reshape(D * S, *output_shape), weight, stride=stride, padding=padding,
                                       output_padding=opad, groups=groups, dilation=dilation)
                    .reshape(D, S, *input_shape))
    if bias is not None:
        bias_map = bias.view(-1, 1, 1).expand(output_shape).reshape(-1)
        delta_u = delta_u + (scaled_u * bias_map).sum(2)
        delta_l = delta_l + (scaled_l * bias_map).sum(2)
    return prev[0], prev[1], delta_u, delta_l
