"""HIP-native CROWN-IBP for chain-structured BoundTask programs.

Host driver mirroring the reference entry points

* ``forward_ibp_trace``        -- boundflow/runtime/crown_ibp.py:101-342 (_forward_ibp_trace_mlp)
* ``run_crown_ibp_mlp``        -- boundflow/runtime/crown_ibp.py:2054-2133
* ``run_crown_ibp_mlp_from_forward_trace`` -- boundflow/runtime/crown_ibp.py:2136-2199
* ``run_crown_all_intermediate`` -- layer-by-layer composition of
  boundflow/runtime/native_intermediate_refinement.py:923-988

with the same argument meaning and error behaviour (ValueError on an
infeasible split or constraint, NotImplementedError for an unsupported graph),
but every numeric step runs in the HIP library on the caller's stream:

* IBP per affine layer in center/radius form (``bf_ibp_linear``), with the
  consumer ReLU's split and constraint intersection fused into the epilogue;
* the CROWN backward as one fused kernel per Affine->ReLU region
  (``bf_crown_relu_linear_fwd``: ReLU relaxation in the A-tile prologue, fp32
  MFMA contraction, bias reductions), and the input layer fused with the
  Linf/box concretization (``bf_crown_relu_linear_concretize``); large queries
  relax each coefficient in the epilogue of the contraction that makes it
  (``bf_crown_relu_linear_relu_fwd``), and queries of few rows relax it in a pass
  of its own (``bf_crown_relu_relax_lu``) ahead of a plain contraction.

Tensors live on the HIP device; nothing is copied to the host except the
feasibility flags when the caller asked for the reference's raise-on-infeasible
behaviour.
"""

from __future__ import annotations

import contextlib
import threading
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Mapping, Optional, Tuple

import torch

from . import _lib
from .profiling import launch as _timed
from .conv import conv_backward_step, ibp_conv2d
from .ir import BFTaskModule, TaskKind
from .spec import BoxPerturbation, InputSpec, IntervalState, LpBallPerturbation, input_norm_p, normalize_input_spec


# ---------------------------------------------------------------------------
# Derived operands kept across queries

_DERIVED: "OrderedDict[tuple, tuple]" = OrderedDict()
_DERIVED_MAX = 64
_SCOPE = threading.local()


def derived(tag: str, sources: Tuple[torch.Tensor, ...], make: Callable[[], torch.Tensor]) -> torch.Tensor:
    """``make()`` of a PARAMETER-derived operand (a layer weight's transpose, a conv bias
    map), computed once per (tag, source tensors) and reused while every source is the
    same tensor object at the same version (no in-place change since), so repeated
    queries skip the copy.  Operands that depend on a query's inputs are never kept here.

    * The entry keeps its sources alive, so their storage cannot be reused under the same
      key; at most 64 entries are kept.  A change written through ``tensor.data`` does not
      bump the version and is not seen: change parameters through the tensor itself.
    * A hit on another stream than the one that made the entry waits for the producer
      (an event recorded after ``make()``), so the consumer never reads it half-written.
    * Inside ``derived_scope()`` (graph capture) entries live in the scope's own dict,
      which the captured query keeps: a replay never reads an entry the process-wide
      cache has since evicted, and ``refresh_scope`` remakes (in place, before a replay)
      every entry whose source changed in place since it was made."""
    scope = getattr(_SCOPE, "memo", None)
    table = _DERIVED if scope is None else scope
    key = (tag,) + tuple(id(t) for t in sources)
    hit = table.get(key)
    versions = tuple(t._version for t in sources)
    if hit is not None and all(a is b for a, b in zip(hit[0], sources)) and hit[1] == versions:
        if scope is None:
            _DERIVED.move_to_end(key)
            out, stream, event = hit[2]
            if event is not None and torch.cuda.current_stream(out.device) != stream:
                torch.cuda.current_stream(out.device).wait_event(event)
            return out
        return hit[2][0]
    out = make()
    stream = event = None
    if scope is None and out.is_cuda:
        stream = torch.cuda.current_stream(out.device)
        event = torch.cuda.Event()
        event.record(stream)
    table[key] = (tuple(sources), versions, (out, stream, event), make if scope is not None else None)
    if scope is None and len(_DERIVED) > _DERIVED_MAX:
        _DERIVED.popitem(last=False)
    return out


@contextlib.contextmanager
def derived_scope(memo: Optional[dict] = None):
    """Route ``derived`` to ``memo`` (a fresh dict when None) for the duration (used
    around graph capture); yields that dict, which the caller keeps as long as the
    captured work may run."""
    prev = getattr(_SCOPE, "memo", None)
    memo = {} if memo is None else memo
    _SCOPE.memo = memo
    try:
        yield memo
    finally:
        _SCOPE.memo = prev


def refresh_scope(memo: dict) -> int:
    """Remake, into the same storage, every entry of a ``derived_scope`` dict whose
    sources changed in place since it was made (in the order the entries were made,
    so an entry derived from another sees the remade one); returns the number remade.
    Runs on the current stream, ahead of whatever is queued after it."""
    n = 0
    with derived_scope(memo):
        for key, (sources, versions, (out, stream, event), make) in list(memo.items()):
            now = tuple(t._version for t in sources)
            if now == versions:
                continue
            out.copy_(make())
            memo[key] = (sources, now, (out, stream, event), make)
            n += 1
    return n


def call_memo(save: Optional[dict], key: str, make: Callable[[], torch.Tensor]) -> torch.Tensor:
    """``make()`` once per optimisation call: per-query operands (scaled gradient rows,
    the first layer's center-plus-bias vector) are kept in the call's own ``save["memo"]``
    dict, which dies with the call, never in the process-wide cache."""
    memo = None if save is None else save.get("memo")
    if memo is None:
        return make()
    out = memo.get(key)
    if out is None:
        out = memo[key] = make()
    return out


def transposed(W: torch.Tensor) -> torch.Tensor:
    """W^T, contiguous (the contraction's faster operand layout), kept across queries."""
    return derived("wt", (W,), lambda: W.t().contiguous())


# ---------------------------------------------------------------------------
# Graph parsing


@dataclass
class AffineLayer:
    kind: str                     # "linear" | "conv2d"
    op_index: int
    in_name: str
    out_name: str
    weight: torch.Tensor
    bias: Optional[torch.Tensor]
    in_shape: Tuple[int, ...]     # per-sample input shape
    out_shape: Tuple[int, ...]    # per-sample output shape
    attrs: Dict[str, object] = field(default_factory=dict)
    relu_input_of_consumer: bool = False   # output feeds a ReLU
    input_is_relu_of: Optional[str] = None  # name of the pre-activation whose ReLU is this layer's input


@dataclass
class Chain:
    layers: List[AffineLayer]
    relu_names: List[str]
    output_value: str

    @property
    def relu_shapes(self) -> Dict[str, Tuple[int, ...]]:
        """Logical (per-example) shape of every ReLU input, in op order."""
        out = {layer.out_name: tuple(layer.out_shape) for layer in self.layers}
        return {name: out[name] for name in self.relu_names}


def _pair(v) -> Tuple[int, int]:
    if isinstance(v, int):
        return (v, v)
    v = tuple(int(x) for x in v)
    return (v[0], v[0]) if len(v) == 1 else (v[0], v[1])


class NotAChain(NotImplementedError):
    """The task is a DAG (a value read by several ops, add, concat, a ReLU not right
    after an affine layer): ``crown_dag`` bounds it with the general backward."""


def parse_chain(module: BFTaskModule, spec: InputSpec, output_value: Optional[str] = None) -> Chain:
    """Validate that the entry task is a chain of affine/ReLU/flatten ops and
    collect per-layer shapes.  Raises NotAChain for DAG structure and
    NotImplementedError for what neither path supports."""
    module.validate()
    task = module.get_entry_task()
    if task.kind != TaskKind.INTERVAL_IBP:
        raise NotImplementedError(f"HIP CROWN only supports INTERVAL_IBP, got {task.kind}")
    if module.task_graph is not None or len(module.tasks) != 1:
        raise NotImplementedError("HIP CROWN supports single-task modules only")
    params = module.params
    if output_value is None:
        if len(task.output_values) != 1:
            raise ValueError(f"task has {len(task.output_values)} outputs; specify output_value explicitly")
        output_value = task.output_values[0]
    shapes: Dict[str, Tuple[int, ...]] = {spec.value_name: tuple(int(d) for d in spec.center.shape[1:])}
    relu_of: Dict[str, str] = {}     # relu output -> relu input
    layers: List[AffineLayer] = []
    relu_names: List[str] = []
    current = spec.value_name
    for idx, op in enumerate(task.ops):
        if len(op.outputs) != 1:
            raise NotImplementedError(f"multi-output op {op.name}")
        x = op.inputs[0]
        t = op.op_type
        if x != current or t in ("add", "concat"):
            raise NotAChain(f"op {op.name} ({t}) makes the task a DAG")
        if t == "linear":
            W = params[op.inputs[1]]
            b = params[op.inputs[2]] if len(op.inputs) == 3 else None
            if W.dim() != 2:
                raise NotImplementedError("batched linear weights are not supported")
            in_shape = shapes[x]
            if len(in_shape) != 1 or in_shape[0] != int(W.shape[1]):
                raise ValueError(f"linear {op.name}: input shape {in_shape} vs weight {tuple(W.shape)}")
            out_shape = (int(W.shape[0]),)
            layers.append(AffineLayer("linear", idx, x, op.outputs[0], W, b, in_shape, out_shape,
                                      input_is_relu_of=relu_of.get(x)))
        elif t == "conv2d":
            W = params[op.inputs[1]]
            b = params[op.inputs[2]] if len(op.inputs) == 3 else None
            in_shape = shapes[x]
            stride = _pair(op.attrs.get("stride", 1))
            padding = _pair(op.attrs.get("padding", 0))
            dilation = _pair(op.attrs.get("dilation", 1))
            groups = int(op.attrs.get("groups", 1))
            if groups != 1 or dilation != (1, 1):
                raise NotImplementedError("HIP conv2d supports groups=1, dilation=1")
            if len(in_shape) != 3 or in_shape[0] != int(W.shape[1]):
                raise ValueError(f"conv2d {op.name}: input shape {in_shape} vs weight {tuple(W.shape)}")
            kh, kw = int(W.shape[2]), int(W.shape[3])
            ho = (in_shape[1] + 2 * padding[0] - kh) // stride[0] + 1
            wo = (in_shape[2] + 2 * padding[1] - kw) // stride[1] + 1
            out_shape = (int(W.shape[0]), ho, wo)
            layers.append(AffineLayer("conv2d", idx, x, op.outputs[0], W, b, in_shape, out_shape,
                                      attrs={"stride": stride, "padding": padding},
                                      input_is_relu_of=relu_of.get(x)))
        elif t == "relu":
            if not layers or layers[-1].out_name != x:
                raise NotAChain("a ReLU that does not follow an affine layer")
            layers[-1].relu_input_of_consumer = True
            relu_of[op.outputs[0]] = x
            relu_names.append(x)
            out_shape = shapes[x]
        elif t in ("flatten", "reshape"):
            if t == "flatten" and (int(op.attrs.get("start_dim", 1)) != 1 or int(op.attrs.get("end_dim", -1)) != -1):
                raise NotImplementedError("flatten(start_dim=1, end_dim=-1) only")
            n = 1
            for d in shapes[x]:
                n *= d
            out_shape = (n,) if t == "flatten" else tuple(int(d) for d in op.attrs["shape"][1:])
            if x in relu_of:
                relu_of[op.outputs[0]] = relu_of[x]
        else:
            raise NotImplementedError(f"HIP CROWN: unsupported op_type {t}")
        if t in ("linear", "conv2d"):
            out_shape = layers[-1].out_shape
        shapes[op.outputs[0]] = out_shape
        current = op.outputs[0]
        if op.outputs[0] == output_value:
            break
    if current != output_value:
        raise ValueError(f"output_value {output_value} not produced by the chain")
    if not layers or layers[-1].out_name != output_value:
        raise NotAChain("the output value is not produced by an affine layer")
    return Chain(layers=layers, relu_names=[r for r in relu_names if r != output_value], output_value=output_value)


def _numel(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


# ---------------------------------------------------------------------------
# Forward IBP trace


@dataclass
class ForwardTrace:
    interval_env: Dict[str, IntervalState]
    relu_pre: Dict[str, IntervalState]
    # int32 [B] (1 = the split/constraint emptied a box); None while no split or constraint
    # was applied (no box can be emptied then): ``infeasible`` makes the zeros on first read
    infeasible_flags: Optional[torch.Tensor]
    input_center_proj: Dict[str, torch.Tensor] = field(default_factory=dict)  # first-layer x0 W^T (no bias)
    batch: int = 0
    device: Optional[torch.device] = None
    # [B, P] radius of a box input, written by the first layer's IBP launch (None: not made there),
    # and the box it was made from: (lower, upper, their versions)
    input_radius: Optional[torch.Tensor] = None
    input_box: Optional[tuple] = None

    @property
    def infeasible(self) -> torch.Tensor:
        if self.infeasible_flags is None:
            self.infeasible_flags = torch.zeros(self.batch, dtype=torch.int32, device=self.device)
        return self.infeasible_flags


def _broadcast_split(split: torch.Tensor, batch: int, numel: int) -> Tuple[torch.Tensor, int]:
    s = split.to(dtype=torch.int8)
    if s.numel() == numel:
        return s.reshape(numel).contiguous(), 0
    if s.numel() == batch * numel and int(s.shape[0]) == batch:
        return s.reshape(batch, numel).contiguous(), numel
    raise ValueError(f"relu split of shape {tuple(split.shape)} cannot broadcast to ({batch}, {numel})")


def forward_ibp_trace(
    module: BFTaskModule,
    input_spec,
    *,
    relu_split_state: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_constraints: Optional[Mapping[str, IntervalState]] = None,
    raise_on_infeasible: bool = True,
    chain: Optional[Chain] = None,
    relu_inputs_only: bool = False,
) -> ForwardTrace:
    """IBP through the chain (crown_ibp.py:101-342).  relu_inputs_only: stop at the
    last layer whose output feeds a ReLU (at least the first layer, whose center
    projection the input region reads); the layers after it get no interval.  A CROWN
    query reads nothing else of the trace: of the output's interval the reference's
    backward reads only its shape (crown_ibp.py:650-669)."""
    spec = normalize_input_spec(input_spec)
    if chain is None:
        try:
            chain = parse_chain(module, spec)
        except NotAChain:
            from .crown_dag import forward_ibp_trace_dag
            return forward_ibp_trace_dag(module, spec, relu_split_state=relu_split_state,
                                         relu_pre_constraints=relu_pre_constraints,
                                         raise_on_infeasible=raise_on_infeasible)
    center = spec.center
    _lib.require_device(center, "input center")
    B = int(center.shape[0])
    dev = center.device
    stream = _lib.stream_handle()
    relu_set = set(chain.relu_names)
    # flags only where a split or a constraint can empty a box (the kernels take NULL)
    may_empty = bool(relu_split_state) or relu_pre_constraints is not None
    infeasible = torch.zeros(B, dtype=torch.int32, device=dev) if may_empty else None
    interval_env: Dict[str, IntervalState] = {}
    relu_pre: Dict[str, IntervalState] = {}
    proj: Dict[str, torch.Tensor] = {}
    pert = spec.perturbation
    norm_p = input_norm_p(pert)
    prev_lo = prev_hi = None
    input_radius = input_box = None
    n_layers = len(chain.layers)
    if relu_inputs_only:
        feeding = [i for i, layer in enumerate(chain.layers) if layer.out_name in relu_set]
        n_layers = (feeding[-1] if feeding else 0) + 1
    for li, layer in enumerate(chain.layers[:n_layers]):
        split = None
        split_ld = 0
        out_numel = _numel(layer.out_shape)
        consumer_relu = layer.out_name in relu_set
        if consumer_relu and relu_split_state is not None and layer.out_name in relu_split_state:
            split, split_ld = _broadcast_split(relu_split_state[layer.out_name].to(dev), B, out_numel)
        has_constraint = consumer_relu and relu_pre_constraints is not None
        lo = torch.empty((B,) + layer.out_shape, device=dev, dtype=torch.float32)
        hi = torch.empty_like(lo)
        first = li == 0
        if layer.kind == "linear":
            K = _numel(layer.in_shape)
            N = out_numel
            ws = torch.empty(int(_lib.load().bf_ibp_linear_workspace(B, K, N)), device=dev, dtype=torch.float32)
            W = layer.weight.contiguous()
            b = None if layer.bias is None else layer.bias.contiguous()
            cproj = None
            if first:
                cproj = torch.empty(B, N, device=dev, dtype=torch.float32)
                if isinstance(pert, BoxPerturbation):
                    in_lo, in_hi, kind, eps, relu_in = (pert.lower.reshape(B, K).contiguous(),
                                                        pert.upper.reshape(B, K).contiguous(), 0, 0.0, 0)
                    # the box radius the input concretization weighs by, written by this launch
                    input_radius = torch.empty(B, K, device=dev, dtype=torch.float32)
                    input_box = (pert.lower, pert.upper, pert.lower._version, pert.upper._version)
                else:
                    # Lp ball: x0 W^T -/+ eps * row norm of W (sum |W|, ||W||_2, max |W| for p = inf, 2, 1)
                    kind = {0: 1, 2: 2, 1: 3}[norm_p]
                    in_lo, in_hi, eps, relu_in = center.reshape(B, K).contiguous(), None, float(pert.eps), 0
            else:
                in_lo, in_hi, kind, eps = prev_lo.reshape(B, K), prev_hi.reshape(B, K), 0, 0.0
                relu_in = 1 if layer.input_is_relu_of is not None else 0
            _lib.call("bf_ibp_linear", _lib.ptr(in_lo), _lib.ptr(in_hi), B, K, kind, eps, relu_in, _lib.ptr(W),
                      _lib.ptr(b), N, _lib.ptr(None if has_constraint else split), split_ld, _lib.ptr(ws),
                      _lib.ptr(lo), _lib.ptr(hi), _lib.ptr(cproj), _lib.ptr(infeasible),
                      _lib.ptr(input_radius if first else None), stream)
            if cproj is not None:
                proj[layer.out_name] = cproj
        else:
            linf = None
            cproj = None
            if first:
                cproj = torch.empty((B,) + layer.out_shape, device=dev, dtype=torch.float32)
                if isinstance(pert, BoxPerturbation):
                    in_lo, in_hi, relu_in = pert.lower.contiguous(), pert.upper.contiguous(), 0
                else:
                    in_lo, in_hi, relu_in, linf = center.contiguous(), None, 0, float(pert.eps)
            else:
                in_lo, in_hi = prev_lo, prev_hi
                relu_in = 1 if layer.input_is_relu_of is not None else 0
            ibp_conv2d(in_lo, in_hi, relu_in, layer, None if has_constraint else split, split_ld, lo, hi,
                       infeasible, linf_eps=linf, center_out=cproj)
            if cproj is not None:
                proj[layer.out_name] = cproj.reshape(B, out_numel)
        if has_constraint:
            c = relu_pre_constraints[layer.out_name]
            _lib.call("bf_interval_clip", _lib.ptr(lo), _lib.ptr(hi), _lib.ptr(c.lower.contiguous()),
                      _lib.ptr(c.upper.contiguous()), _lib.ptr(split), split_ld, B, out_numel,
                      _lib.ptr(infeasible), stream)
        st = IntervalState(lo, hi)
        interval_env[layer.out_name] = st
        if consumer_relu:
            relu_pre[layer.out_name] = st
        prev_lo, prev_hi = lo, hi
    if raise_on_infeasible and (relu_split_state or relu_pre_constraints):
        if bool(infeasible.any().item()):
            raise ValueError("infeasible relu split or constraint: lower>upper after applying split")
    return ForwardTrace(interval_env=interval_env, relu_pre=relu_pre, infeasible_flags=infeasible, batch=B, device=dev,
                        input_center_proj=proj, input_radius=input_radius, input_box=input_box)


# ---------------------------------------------------------------------------
# CROWN backward


def _flat_param(v: torch.Tensor, batch: int, numel: int, label: str) -> Tuple[torch.Tensor, int]:
    """[*shape] / [numel] / [1, numel] -> shared (stride 0); [B, *shape] -> per-domain (stride numel)."""
    v = v.to(torch.float32)
    if v.numel() == numel:
        return v.reshape(numel).contiguous(), 0
    if v.numel() == batch * numel and int(v.shape[0]) == batch:
        return v.reshape(batch, numel).contiguous(), numel
    raise ValueError(f"{label} of shape {tuple(v.shape)} cannot broadcast to ({batch}, {numel})")


@dataclass
class BackwardSaved:
    """Per-layer tensors kept for the gradient pass (lower bound only)."""
    A_in: List[Optional[torch.Tensor]]      # coefficient entering each layer's relaxation ([M, n_k]) or None
    b_rows: torch.Tensor


def _init_spec(C: Optional[torch.Tensor], batch: int, out_dim: int, dev) -> Tuple[torch.Tensor, int, int]:
    """Return (A0, S, a_dstride) for the initial coefficient (crown_ibp.py:672-719)."""
    if C is None:
        eye = torch.eye(out_dim, device=dev, dtype=torch.float32)
        return eye, out_dim, 0
    C = C.to(device=dev, dtype=torch.float32)
    if C.dim() == 2:
        if int(C.shape[1]) != out_dim:
            raise ValueError(f"linear_spec_C shape mismatch: C={tuple(C.shape)} out=({batch}, {out_dim})")
        return C.contiguous(), int(C.shape[0]), 0
    if C.dim() != 3 or int(C.shape[0]) != batch or int(C.shape[2]) != out_dim:
        raise ValueError(f"linear_spec_C shape mismatch: C={tuple(C.shape)} out=({batch}, {out_dim})")
    S = int(C.shape[1])
    return C.contiguous(), S, S * out_dim


def crown_backward(
    module: BFTaskModule,
    spec: InputSpec,
    trace: ForwardTrace,
    *,
    chain: Chain,
    linear_spec_C: Optional[torch.Tensor] = None,
    relu_alpha: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_add_coeff_l: Optional[Dict[str, torch.Tensor]] = None,
    need_upper: bool = True,
    need_lower: bool = True,
    save: Optional[dict] = None,
) -> IntervalState:
    dev = spec.center.device
    B = int(spec.center.shape[0])
    stream = _lib.stream_handle()
    layers = chain.layers
    out_dim = _numel(layers[-1].out_shape)
    A0, S, a_dstride = _init_spec(linear_spec_C, B, out_dim, dev)
    M = B * S
    pert = spec.perturbation
    A_u: Optional[torch.Tensor] = A0 if need_upper else None
    A_l: Optional[torch.Tensor] = A0 if need_lower else None
    b_u = b_l = None
    c_u = c_l = None
    stride = a_dstride
    tables: Dict[int, torch.Tensor] = {}

    def relax_params(k: int):
        """(alpha, alpha_ld, add, add_ld, pre_lo, pre_hi, N) of the ReLU after layer k."""
        layer = layers[k]
        relax_name = layer.out_name if k < len(layers) - 1 else None
        pre = trace.relu_pre[relax_name] if relax_name is not None else None
        n = _numel(layer.out_shape)
        alpha = add = None
        alpha_ld = add_ld = 0
        if relax_name is not None:
            if relu_alpha is not None and relax_name in relu_alpha:
                alpha, alpha_ld = _flat_param(relu_alpha[relax_name], B, n, f"relu_alpha[{relax_name}]")
            if relu_pre_add_coeff_l is not None and relax_name in relu_pre_add_coeff_l:
                add, add_ld = _flat_param(relu_pre_add_coeff_l[relax_name], B, n,
                                          f"relu_pre_add_coeff_l[{relax_name}]")
        pre_lo = None if pre is None else pre.lower.reshape(B, n)
        pre_hi = None if pre is None else pre.upper.reshape(B, n)
        return alpha, alpha_ld, add, add_ld, pre_lo, pre_hi, n

    def relax_table(k: int) -> Optional[torch.Tensor]:
        """Slopes/intercepts of the ReLU after linear layer k, once per (domain, neuron), shared by both bounds."""
        if k in tables:
            return tables[k]
        # A query of many rows reads the tables of every linear layer below this one in
        # turn: they are built together, in one launch.
        todo = [j for j in range(k, -1, -1) if j not in tables] if M >= EPILOGUE_MIN_M else [k]
        built = []
        for j in todo:
            alpha, alpha_ld, _, _, pre_lo, pre_hi, n = relax_params(j)
            table = None
            if pre_lo is not None and layers[j].kind == "linear":
                table = torch.empty(B, n, 4, device=dev, dtype=torch.float32)
                built.append((pre_lo, pre_hi, alpha, alpha_ld, n, table))
            tables[j] = table
        if len(built) == 1:
            pre_lo, pre_hi, alpha, alpha_ld, n, table = built[0]
            _lib.call("bf_relu_relax_table", _lib.ptr(pre_lo), _lib.ptr(pre_hi), _lib.ptr(alpha), alpha_ld, B, n,
                      _lib.ptr(table), stream)
        elif built:
            col = lambda i: [t[i] for t in built]
            _lib.call("bf_relu_relax_table_multi", len(built), _lib.ptr_array(col(0)), _lib.ptr_array(col(1)),
                      _lib.ptr_array(col(2)), _lib.i64_array(col(3)), B, _lib.i64_array(col(4)),
                      _lib.ptr_array(col(5)), stream)
        return tables[k]

    # A coefficient produced by bf_crown_relu_linear_relu_fwd already carries the
    # relaxation (and bias) of the ReLU it enters: the next region skips its prologue.
    pre_relaxed = False
    relax_pass_next = False   # the coefficient is a kept head product: relax it in a pass of its own
    for k in range(len(layers) - 1, -1, -1):
        layer = layers[k]
        alpha, alpha_ld, add, add_ld, pre_lo, pre_hi, N = relax_params(k)
        # the relaxation of this region is still to apply (its table is built on first use)
        relaxes = pre_lo is not None and layer.kind == "linear" and not pre_relaxed
        if pre_relaxed:
            add = None
            add_ld = 0
        if save is not None and A_l is not None and not pre_relaxed:
            # (a coefficient relaxed by the producing epilogue had its unrelaxed form recorded there)
            save.setdefault("A_in", {})[k] = (A_l, stride)
            save.setdefault("b_in", {})[k] = b_l
        if layer.kind == "conv2d":
            relax_pass_next = False   # a conv region relaxes its coefficient itself
            A_u, A_l, b_u, b_l, stride, done = conv_backward_step(
                layer, k == 0, A_u, A_l, stride, b_u, b_l, B, S, pre_lo, pre_hi, alpha, alpha_ld, add, add_ld,
                spec, trace, save=save)
            if done is not None:
                return done
            continue
        W = layer.weight.contiguous()
        # the contraction reads W^T [P, N] row-major: 128-bit operand loads along N
        Wt = transposed(W)
        bias = None if layer.bias is None or pre_relaxed else layer.bias.contiguous()
        P = _numel(layer.in_shape)
        if k > 0 and linear_spec_C is None and k == len(layers) - 1:
            # C = I: I @ W is W itself, shared by every domain (no contraction needed)
            A_u = W if A_u is not None else None
            A_l = W if A_l is not None else None
            brow = (bias if bias is not None else torch.zeros(N, device=dev)).repeat(B).contiguous()
            b_u = brow if A_u is not None else None
            b_l = brow if A_l is not None else None
            stride = 0
            continue
        shared_first = (stride == 0 and S >= EPILOGUE_MIN_ROWS and M >= EPILOGUE_MIN_M
                        and (k == 0 or layers[k - 1].kind == "linear"))
        small_grid = M < EPILOGUE_MIN_M and N >= RELAX_PASS_MIN_K
        if relaxes and (shared_first or small_grid or relax_pass_next):
            # A coefficient shared by every domain (the first region of a C = I query):
            # its relaxation differs per domain, so one bandwidth-bound pass writes it
            # per domain (with the bias terms and, at the input layer, the center sums)
            # and the contraction below runs with the plain prologue.  A query of few
            # rows takes the same two steps: its contraction is a grid of few tiles whose
            # K loop runs serially on a few CUs, and the plain prologue deals it as
            # 64 x 64 tiles over four times as many CUs as the relaxation prologue's
            # 128 x 128 ones.
            cvec0 = trace.input_center_proj.get(layer.out_name) if k == 0 else None
            if k == 0 and cvec0 is None:
                raise RuntimeError("forward trace lacks the input-layer projection")
            rA_u = torch.empty(M, N, device=dev, dtype=torch.float32) if A_u is not None else None
            rA_l = torch.empty(M, N, device=dev, dtype=torch.float32) if A_l is not None else None
            rb_u = torch.empty(M, device=dev, dtype=torch.float32) if A_u is not None else None
            rb_l = torch.empty(M, device=dev, dtype=torch.float32) if A_l is not None else None
            c_u = torch.empty(M, device=dev, dtype=torch.float32) if (cvec0 is not None and A_u is not None) else None
            c_l = torch.empty(M, device=dev, dtype=torch.float32) if (cvec0 is not None and A_l is not None) else None
            nz = int(A_u is not None) + int(A_l is not None)
            with _timed("crown_relu_relax", 0.0, 4.0 * nz * ((M if stride else S) * N + M * N)):
                _lib.call("bf_crown_relu_relax_lu", _lib.ptr(A_u), _lib.ptr(A_l), stride, B, S, N, _lib.ptr(pre_lo),
                          _lib.ptr(pre_hi), _lib.ptr(alpha), alpha_ld, _lib.ptr(add), add_ld, _lib.ptr(bias),
                          _lib.ptr(cvec0), _lib.ptr(b_u), _lib.ptr(b_l), _lib.ptr(rA_u), _lib.ptr(rA_l),
                          _lib.ptr(rb_u), _lib.ptr(rb_l), _lib.ptr(c_u), _lib.ptr(c_l), stream)
            A_u, A_l, b_u, b_l = rA_u, rA_l, rb_u, rb_l
            stride = S * N
            add = bias = None
            add_ld = 0
            relaxes = False
            pre_relaxed = True
        relax_pass_next = False
        relax = relax_table(k) if relaxes else None
        if k == 0 and pre_relaxed:
            # input layer of an already relaxed coefficient: contraction fused with the concretization
            rad, eps = _input_radius(pert, B, P, trace)
            ws = torch.empty(int(_lib.load().bf_crown_linear_concretize_workspace(B, S, P)), device=dev,
                             dtype=torch.float32)
            lb = torch.empty(B, S, device=dev, dtype=torch.float32) if A_l is not None else None
            ub = torch.empty(B, S, device=dev, dtype=torch.float32) if A_u is not None else None
            h_scale = h_out = None
            if save is not None and save.get("grad_rows") is not None:
                # gradient seed of the concretization: h = -eps * G * sign(A W) (* radius for a box)
                h_scale = call_memo(save, f"h_scale:{eps!r}", lambda: (save["grad_rows"] * (-eps)).contiguous())
                h_out = torch.empty(M, P, device=dev, dtype=torch.float32)
                save["h"] = h_out
                save["cvec"] = trace.input_center_proj.get(layer.out_name)
            nz = int(A_u is not None) + int(A_l is not None)
            # bytes: the coefficient rows and the weight read, the row partial norms written, the
            # gradient seed [M, P] written when asked
            with _timed("crown_linear_concretize", 2.0 * nz * M * N * P,
                        4.0 * nz * (M * N + N * P + M * -(-P // 128)) + (4.0 * M * P if h_out is not None else 0.0)):
                _lib.call("bf_crown_linear_concretize", _lib.ptr(A_u), _lib.ptr(A_l), stride, B, S, N, _lib.ptr(Wt),
                          P, _lib.ptr(rad), eps, input_norm_p(pert), _lib.ptr(c_u), _lib.ptr(c_l), _lib.ptr(b_u),
                          _lib.ptr(b_l),
                          _lib.ptr(h_scale), _lib.ptr(h_out), _lib.ptr(ws), _lib.ptr(lb), _lib.ptr(ub), stream)
            if save is not None:
                save["final_ws"] = ws
            return IntervalState(lower=lb, upper=ub)
        if k == 0:
            # input layer: relaxation + contraction fused with the concretization
            if isinstance(pert, BoxPerturbation):
                rad = _input_radius(pert, B, P, trace)[0]
                cvec = trace.input_center_proj.get(layer.out_name)
                # center term A' (mid W^T): the trace holds mid W^T when the input is a box
                eps = 1.0
            else:
                rad = None
                cvec = trace.input_center_proj.get(layer.out_name)
                eps = float(pert.eps)
            if cvec is None:
                raise RuntimeError("forward trace lacks the input-layer projection")
            ws = torch.empty(int(_lib.load().bf_crown_relu_linear_concretize_workspace(B, S, P)), device=dev,
                             dtype=torch.float32)
            lb = torch.empty(B, S, device=dev, dtype=torch.float32) if A_l is not None else None
            ub = torch.empty(B, S, device=dev, dtype=torch.float32) if A_u is not None else None
            h_scale = h_out = None
            if save is not None and save.get("grad_rows") is not None:
                # gradient seed of the concretization: h = -eps * G * sign(A W) (* radius for a box)
                h_scale = call_memo(save, f"h_scale:{eps!r}", lambda: (save["grad_rows"] * (-eps)).contiguous())
                h_out = torch.empty(M, P, device=dev, dtype=torch.float32)
                save["h"] = h_out
                save["cvec"] = cvec
            nz = int(A_u is not None) + int(A_l is not None)
            with _timed("crown_relu_linear_concretize", 2.0 * nz * M * N * P,
                        4.0 * nz * (M * N + N * P) + 16.0 * B * N + (4.0 * M * P if h_out is not None else 0.0)):
                _lib.call("bf_crown_relu_linear_concretize", _lib.ptr(A_u), _lib.ptr(A_l), stride, B, S, N,
                          _lib.ptr(relax), _lib.ptr(add), add_ld, _lib.ptr(Wt), P, 1, _lib.ptr(bias), _lib.ptr(cvec),
                          _lib.ptr(rad), eps, input_norm_p(pert), _lib.ptr(b_u),
                          _lib.ptr(b_l), _lib.ptr(h_scale), _lib.ptr(h_out), _lib.ptr(ws), _lib.ptr(lb),
                          _lib.ptr(ub), stream)
            if save is not None:
                save["final_ws"] = ws
            return IntervalState(lower=lb, upper=ub)
        nA_u = torch.empty(M, P, device=dev, dtype=torch.float32) if A_u is not None else None
        nA_l = torch.empty(M, P, device=dev, dtype=torch.float32) if A_l is not None else None
        nb_u = torch.empty(M, device=dev, dtype=torch.float32) if A_u is not None else None
        nb_l = torch.empty(M, device=dev, dtype=torch.float32) if A_l is not None else None
        nz = int(A_u is not None) + int(A_l is not None)
        a_rows = M if stride != 0 else S
        flops, nbytes = 2.0 * nz * M * N * P, 4.0 * nz * (a_rows * N + N * P + M * P)
        # The head region (the spec C through the last layer, nothing to relax) depends on C
        # and the layer's parameters alone: an optimisation call makes it once and its later
        # passes reuse it (kept in the call's own memo, keyed by C's storage and version); the
        # next region then relaxes the kept product in a pass of its own.
        head_memo = (k == len(layers) - 1 and relax is None and add is None and save is not None
                     and save.get("memo") is not None and torch.is_tensor(linear_spec_C))
        if not head_memo and layers[k - 1].kind == "linear" and S >= EPILOGUE_MIN_ROWS and M >= EPILOGUE_MIN_M:
            # the next region's relaxation in this contraction's epilogue
            n_alpha, n_alpha_ld, n_add, n_add_ld, _, _, _ = relax_params(k - 1)
            n_table = relax_table(k - 1)
            prev = layers[k - 1]
            n_bias = None if prev.bias is None else prev.bias.contiguous()
            cvec = None
            if k - 1 == 0:
                cvec = trace.input_center_proj.get(prev.out_name)
                if cvec is None:
                    raise RuntimeError("forward trace lacks the input-layer projection")
            if n_table is None:
                n_table = _identity_table(B, P, dev)
            ws = torch.empty(int(_lib.load().bf_crown_relu_linear_relu_fwd_workspace(B, S, P)), device=dev,
                             dtype=torch.float32)
            nc_u = torch.empty(M, device=dev, dtype=torch.float32) if (cvec is not None and A_u is not None) else None
            nc_l = torch.empty(M, device=dev, dtype=torch.float32) if (cvec is not None and A_l is not None) else None
            # the gradient pass reads the lower coefficient before the next relaxation
            pre_l = torch.empty(M, P, device=dev, dtype=torch.float32) if (save is not None and A_l is not None) else None
            # bytes: the next relaxation's operands per (domain, column) -- the float4 table, the split
            # term of the lower bound, the center projection -- and the row partial sums are read or
            # written once; the unrelaxed lower coefficient kept for the gradient is a second output
            e_bytes = (16.0 * B * P + (4.0 * B * P if (n_add is not None and A_l is not None) else 0.0)
                       + (4.0 * B * P if cvec is not None else 0.0)
                       + 4.0 * nz * M * -(-P // 128) * (2 if cvec is not None else 1))
            with _timed("crown_relu_linear_relu_fwd", flops,
                        nbytes + e_bytes + (4.0 * M * P if pre_l is not None else 0.0)):
                _lib.call("bf_crown_relu_linear_relu_fwd", _lib.ptr(A_u), _lib.ptr(A_l), stride, B, S, N,
                          _lib.ptr(relax), _lib.ptr(add), add_ld, _lib.ptr(Wt), P, _lib.ptr(bias), _lib.ptr(b_u),
                          _lib.ptr(b_l), _lib.ptr(n_table), _lib.ptr(n_add), n_add_ld, _lib.ptr(n_bias),
                          _lib.ptr(cvec), P, _lib.ptr(ws), _lib.ptr(nA_u), _lib.ptr(nA_l), None, _lib.ptr(pre_l),
                          _lib.ptr(nb_u), _lib.ptr(nb_l), _lib.ptr(nc_u), _lib.ptr(nc_l), stream)
            if pre_l is not None:
                save.setdefault("A_in", {})[k - 1] = (pre_l, S * P)
                save.setdefault("b_in", {})[k - 1] = nb_l
            c_u, c_l = nc_u, nc_l
            pre_relaxed = True
        else:
            # with nothing to relax and no bias the contraction leaves the bias rows as they
            # are: they pass through instead of being copied
            keep_b = (relax is None and add is None and bias is None and (A_u is None or b_u is not None)
                      and (A_l is None or b_l is not None))
            if keep_b:
                nb_u, nb_l = b_u, b_l
            head_key = None
            if head_memo:
                head_key = (f"head:{k}:{linear_spec_C.data_ptr()}:{linear_spec_C._version}:"
                            f"{A_u is not None}:{A_l is not None}")
                relax_pass_next = True
            hit = save["memo"].get(head_key) if head_key is not None else None
            if hit is not None:
                nA_u, nA_l, nb_u, nb_l = hit
            else:
                with _timed("crown_relu_linear_fwd", flops, nbytes):
                    _lib.call("bf_crown_relu_linear_fwd", _lib.ptr(A_u), _lib.ptr(A_l), stride, B, S, N,
                              _lib.ptr(relax), _lib.ptr(add), add_ld, _lib.ptr(Wt), P, 1, _lib.ptr(bias),
                              None if keep_b else _lib.ptr(b_u), None if keep_b else _lib.ptr(b_l), _lib.ptr(nA_u),
                              _lib.ptr(nA_l), None if keep_b else _lib.ptr(nb_u), None if keep_b else _lib.ptr(nb_l),
                              stream)
                if head_key is not None:
                    save["memo"][head_key] = (nA_u, nA_l, nb_u, nb_l)
            pre_relaxed = False
        A_u, A_l, b_u, b_l = nA_u, nA_l, nb_u, nb_l
        stride = S * P
    raise RuntimeError("backward did not reach the input layer")


# The backward relaxes each coefficient in the epilogue of the contraction that
# produces it when a domain has at least EPILOGUE_MIN_ROWS rows (a 128-row tile then
# spans at most 17 domains, whose relaxation entries fit the LDS stage of the
# library's choice of tile) and the query has at least EPILOGUE_MIN_M rows (below
# that, the launch-bound query is better served by the fewer launches of the fused
# prologue).
EPILOGUE_MIN_ROWS = 8
EPILOGUE_MIN_M = 8192

# A query below EPILOGUE_MIN_M rows relaxes a coefficient of at least this many
# columns in a pass of its own before the contraction (plain prologue); narrower
# coefficients keep the fused prologue, whose K loop is then one or two tiles long.
RELAX_PASS_MIN_K = 32


def _identity_table(B: int, n: int, dev) -> torch.Tensor:
    """Relaxation table of a linear (no ReLU) boundary: slopes 1, intercepts 0."""
    t = torch.zeros(B, n, 4, device=dev, dtype=torch.float32)
    t[:, :, 0] = 1.0
    t[:, :, 2] = 1.0
    return t


def _input_radius(pert, B: int, P: int, trace=None):
    """(rad, eps) of the input concretization: box radius with eps 1, or Linf eps without weights.
    The radius the trace's first IBP launch wrote when it was made from this very box (same
    tensors, unchanged since), else one launch here."""
    if isinstance(pert, BoxPerturbation):
        box = getattr(trace, "input_box", None)
        if (box is not None and box[0] is pert.lower and box[1] is pert.upper
                and box[2] == pert.lower._version and box[3] == pert.upper._version):
            return trace.input_radius, 1.0
        lo = pert.lower.reshape(B, P).contiguous()
        hi = pert.upper.reshape(B, P).contiguous()
        # depends on the query's input set: computed per query (one launch), never kept across queries
        rad = torch.empty(B, P, device=lo.device, dtype=torch.float32)
        _lib.call("bf_interval_center_radius", _lib.ptr(lo), _lib.ptr(hi), B * P, 0, None, _lib.ptr(rad),
                  _lib.stream_handle())
        return rad, 1.0
    return None, float(pert.eps)


def _with_upper_add(backward, relu_pre, C, add_l, add_u, B: int, out_dim: int) -> IntervalState:
    """Both bounds with the split terms of the lower (``add_l``) and upper (``add_u``)
    coefficients.  With ``add_u`` (crown_ibp.py:1270-1278: added to A_u after its
    relaxation, rank-2 pre-activations only, :1256-1260) the upper bound is minus the
    lower bound of -C with the term -add_u: every step of that pass is the upper pass's
    arithmetic with each value negated (the relaxation select A >= 0 differs only where
    A = 0, whose products are zero), so its results are the upper pass's, negated."""
    if not add_u:
        return backward(C, add_l, True, True)
    for name, v in add_u.items():
        pre = relu_pre.get(name)
        if pre is not None and pre.lower.dim() != 2:
            raise NotImplementedError(
                f"run_crown_ibp_mlp only supports relu_pre_add_coeff_u on rank-2 pre-activations; got "
                f"{tuple(pre.lower.shape)} for {name}")
    if C is None:
        dev = next(iter(relu_pre.values())).lower.device if relu_pre else None
        C = torch.eye(out_dim, device=dev).unsqueeze(0).expand(B, out_dim, out_dim).contiguous()
    lower = backward(C, add_l, False, True).lower
    neg_add = {k: -v for k, v in add_u.items()}
    upper = -backward(-C, neg_add, False, True).lower
    return IntervalState(lower=lower, upper=upper)


def run_crown_ibp_mlp(
    module: BFTaskModule,
    input_spec,
    *,
    linear_spec_C: Optional[torch.Tensor] = None,
    output_value: Optional[str] = None,
    relu_alpha: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_add_coeff_u: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_add_coeff_l: Optional[Dict[str, torch.Tensor]] = None,
    relu_split_state: Optional[Dict[str, torch.Tensor]] = None,
) -> IntervalState:
    """HIP counterpart of run_crown_ibp_mlp (crown_ibp.py:2054-2133).  Chains run the
    fused region kernels; DAG tasks (add, concat, fan-out) the general backward of
    ``crown_dag``."""
    spec = normalize_input_spec(input_spec)
    try:
        chain_full = parse_chain(module, spec)
    except NotAChain:
        from .crown_dag import forward_ibp_trace_dag
        trace = forward_ibp_trace_dag(module, spec, relu_split_state=relu_split_state)
        return run_crown_ibp_mlp_from_forward_trace(module, spec, trace=trace, linear_spec_C=linear_spec_C,
                                                    output_value=output_value, relu_alpha=relu_alpha,
                                                    relu_pre_add_coeff_u=relu_pre_add_coeff_u,
                                                    relu_pre_add_coeff_l=relu_pre_add_coeff_l)
    trace = forward_ibp_trace(module, spec, relu_split_state=relu_split_state, chain=chain_full,
                              relu_inputs_only=True)
    chain = parse_chain(module, spec, output_value) if output_value is not None else chain_full

    def backward(C, add_l, need_upper, need_lower):
        return crown_backward(module, spec, trace, chain=chain, linear_spec_C=C, relu_alpha=relu_alpha,
                              relu_pre_add_coeff_l=add_l, need_upper=need_upper, need_lower=need_lower)

    return _with_upper_add(backward, trace.relu_pre, linear_spec_C, relu_pre_add_coeff_l, relu_pre_add_coeff_u,
                           int(spec.center.shape[0]), _numel(chain.layers[-1].out_shape))


def run_crown_ibp_mlp_from_forward_trace(
    module: BFTaskModule,
    input_spec,
    *,
    trace: ForwardTrace,
    linear_spec_C: Optional[torch.Tensor] = None,
    output_value: Optional[str] = None,
    relu_alpha: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_add_coeff_u: Optional[Dict[str, torch.Tensor]] = None,
    relu_pre_add_coeff_l: Optional[Dict[str, torch.Tensor]] = None,
) -> IntervalState:
    """HIP counterpart of run_crown_ibp_mlp_from_forward_trace (crown_ibp.py:2136-2199)."""
    spec = normalize_input_spec(input_spec)
    from .crown_dag import DagTrace, crown_backward_dag
    B = int(spec.center.shape[0])
    if isinstance(trace, DagTrace):
        out = output_value or module.get_entry_task().output_values[0]

        def backward(C, add_l, need_upper, need_lower):
            return crown_backward_dag(module, spec, trace, linear_spec_C=C, output_value=output_value,
                                      relu_alpha=relu_alpha, relu_pre_add_coeff_l=add_l, need_upper=need_upper,
                                      need_lower=need_lower)

        return _with_upper_add(backward, trace.relu_pre, linear_spec_C, relu_pre_add_coeff_l, relu_pre_add_coeff_u,
                               B, _numel(trace.shapes[out]))
    chain = parse_chain(module, spec, output_value)

    def backward(C, add_l, need_upper, need_lower):
        return crown_backward(module, spec, trace, chain=chain, linear_spec_C=C, relu_alpha=relu_alpha,
                              relu_pre_add_coeff_l=add_l, need_upper=need_upper, need_lower=need_lower)

    return _with_upper_add(backward, trace.relu_pre, linear_spec_C, relu_pre_add_coeff_l, relu_pre_add_coeff_u, B,
                           _numel(chain.layers[-1].out_shape))


def run_crown_ibp_mlp_with_relu_influence_from_forward_trace(
    module: BFTaskModule,
    input_spec,
    *,
    interval_env: Dict[str, IntervalState],
    relu_pre: Dict[str, IntervalState],
    linear_spec_C: torch.Tensor,
    output_value: Optional[str] = None,
) -> Tuple[IntervalState, Dict[str, torch.Tensor]]:
    """Bounds of the objective C and each ReLU's objective influence (crown_ibp.py:2201-2241):
    for every ReLU input x, max over the spec rows of max(|A_u|, |A_l|) of the backward
    coefficient of the ReLU's output, [B, *shape of x].  The backward runs on dense rows
    (``crown_dag``) from the given boxes; one INTERVAL_IBP task, as in the reference."""
    from .crown_dag import DagTrace, crown_backward_dag, value_shapes
    module.validate()
    task = module.get_entry_task()
    if task.kind != TaskKind.INTERVAL_IBP:
        raise NotImplementedError("ReLU influence extraction only supports INTERVAL_IBP tasks")
    if module.task_graph is not None or len(module.tasks) != 1:
        raise NotImplementedError("ReLU influence extraction currently supports one task only")
    spec = normalize_input_spec(input_spec)
    shapes, _relu_shapes = value_shapes(module, spec)
    trace = DagTrace(interval_env=dict(interval_env), relu_pre=dict(relu_pre), shapes=shapes,
                     batch=int(spec.center.shape[0]), device=spec.center.device)
    influence: Dict[str, torch.Tensor] = {}
    bounds = crown_backward_dag(module, spec, trace, linear_spec_C=linear_spec_C, output_value=output_value,
                                relu_influence=influence)
    if set(influence) != set(relu_pre):
        raise ValueError("ReLU objective influence coverage differs")
    return bounds, {name: influence[name] for name in relu_pre}


@dataclass
class CrownIbpStats:
    """Whether ``run_crown_ibp_mlp`` takes a module (crown_ibp.py:63-67)."""
    supported: bool
    reason: str = ""
    ops_seen: Tuple[str, ...] = ()


def get_crown_ibp_mlp_stats(module: BFTaskModule) -> CrownIbpStats:
    """The support check of crown_ibp.py:2279-2350 for this path: one INTERVAL_IBP task of
    linear / relu / conv2d / flatten / reshape / add / concat ops (chains and DAGs), with
    single outputs, flatten over (1, -1), two-operand adds, concats of two or more
    operands on the feature or channel axis, and conv2d with groups 1 and dilation 1.
    Never raises: what fails validation is reported as unsupported with the reason."""
    from .crown_dag import DAG_OPS
    try:
        module.validate()
        task = module.get_entry_task()
        if task.kind != TaskKind.INTERVAL_IBP:
            return CrownIbpStats(False, f"TaskKind={task.kind}")
        if module.task_graph is not None or len(module.tasks) != 1:
            return CrownIbpStats(False, "multi-task module not supported")
        ops = tuple(op.op_type for op in task.ops)
        if not ops:
            return CrownIbpStats(False, "empty task", ops)
        bad = [t for t in ops if t not in DAG_OPS]
        if bad:
            return CrownIbpStats(False, f"unsupported ops: {bad}", ops)
        for i, op in enumerate(task.ops):
            t = op.op_type
            if len(op.outputs) != 1:
                return CrownIbpStats(False, f"multi-output op not supported at op {i}: outputs={op.outputs}", ops)
            if t == "flatten" and (int(op.attrs.get("start_dim", 1)), int(op.attrs.get("end_dim", -1))) != (1, -1):
                return CrownIbpStats(False, f"unsupported flatten attrs at op {i}: {op.attrs}", ops)
            if t == "add" and len(op.inputs) != 2:
                return CrownIbpStats(False, f"add expects 2 inputs at op {i}, got {len(op.inputs)}", ops)
            if t == "concat":
                if len(op.inputs) < 2:
                    return CrownIbpStats(False, f"concat expects at least 2 inputs at op {i}, got {len(op.inputs)}",
                                         ops)
                if int(op.attrs.get("axis", 1)) not in (1, -1):
                    return CrownIbpStats(False, f"unsupported concat axis at op {i}: {op.attrs.get('axis', 1)}", ops)
            if t == "conv2d":
                dilation = _pair(op.attrs.get("dilation", 1))
                if int(op.attrs.get("groups", 1)) != 1 or dilation != (1, 1):
                    return CrownIbpStats(False, f"conv2d with groups or dilation != 1 at op {i}", ops)
        return CrownIbpStats(True, "", ops)
    except Exception as e:   # validation errors are the answer, not a failure of the check
        return CrownIbpStats(False, str(e))


def run_crown_all_intermediate(module: BFTaskModule, input_spec, *, linear_spec_C: torch.Tensor):
    """Every intermediate pre-activation bound by CROWN (C = I per layer),
    intersected with the IBP bound, then the final spec bound; the composition of
    native_intermediate_refinement.py:923-988 applied to every ReLU after the first."""
    spec = normalize_input_spec(input_spec)
    chain_full = parse_chain(module, spec)
    trace = forward_ibp_trace(module, spec, chain=chain_full, relu_inputs_only=True)
    names = list(trace.relu_pre.keys())
    stream = _lib.stream_handle()
    B = int(spec.center.shape[0])
    for name in names[1:]:
        chain = parse_chain(module, spec, name)
        b = crown_backward(module, spec, trace, chain=chain, linear_spec_C=None)
        cur = trace.relu_pre[name]
        n = int(cur.lower[0].numel())
        lo = cur.lower.reshape(B, n)
        hi = cur.upper.reshape(B, n)
        flag = torch.zeros(B, dtype=torch.int32, device=spec.center.device)
        _lib.call("bf_interval_clip", _lib.ptr(lo), _lib.ptr(hi), _lib.ptr(b.lower.contiguous()),
                  _lib.ptr(b.upper.contiguous()), None, 0, B, n, _lib.ptr(flag), stream)
    final = crown_backward(module, spec, trace, chain=chain_full, linear_spec_C=linear_spec_C)
    return final, trace.relu_pre
