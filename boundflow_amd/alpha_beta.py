"""HIP alpha-CROWN / alpha-beta-CROWN optimisation loop.

Mirrors ``run_alpha_beta_crown_mlp`` (boundflow/runtime/alpha_beta_crown.py:643-941)
and ``run_alpha_crown_mlp`` (boundflow/runtime/alpha_crown.py:137-261) for the
"lower" objective with the "mean" spec reduction, the configuration the BaB
solver uses (boundflow/runtime/bab.py:134-153):

* one forward IBP trace (split-aware), branch choices from it
  (alpha_beta_crown.py:145-182);
* ``steps + 1`` evaluations of the lower bound (the fused CROWN backward keeps
  the coefficients the gradient needs);
* best-of tracking per domain (per_batch_params) or globally, then one upper
  bound evaluation with the best parameters;
* between evaluations, the analytic reverse pass of the lower bound (the
  gradient autograd computes in the reference): fused concretization seed ->
  transposed contractions with rank-1 bias terms -> per-ReLU gradient kernels
  that reduce dL/dalpha and dL/dbeta over the specs;
* torch.optim.Adam's update (lr, betas 0.9/0.999, eps 1e-8) and the clamps
  alpha in [0, 1], beta >= 0, applied in place on the device.

The loss is -sum_d mean_s lb (per-domain parameters) or -mean lb (shared), so
the gradient of every lower bound row is -1/S or -1/(D*S).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Tuple

import numpy as np
import torch

from . import _lib
from .crown import (
    Chain,
    ForwardTrace,
    _broadcast_split,
    _numel,
    call_memo,
    crown_backward,
    derived,
    forward_ibp_trace,
    NotAChain,
    parse_chain,
)
from .profiling import launch as _timed
from .spec import InputSpec, IntervalState, normalize_input_spec


class AlphaState(dict):
    """Alpha per ReLU input (alpha_crown.py:25-30): a dict of ReLU input name to the
    slopes, which ``alpha_by_relu_input`` also returns, so the reference's and this
    package's callers read it alike."""

    @property
    def alpha_by_relu_input(self) -> Dict[str, torch.Tensor]:
        return self

    def detach_clone(self) -> "AlphaState":
        return AlphaState({k: v.detach().clone() for k, v in self.items()})


class BetaState(dict):
    """Beta per ReLU input (alpha_beta_crown.py:29-42), as AlphaState."""

    @property
    def beta_by_relu_input(self) -> Dict[str, torch.Tensor]:
        return self

    def detach_clone(self) -> "BetaState":
        return BetaState({k: v.detach().clone() for k, v in self.items()})


def _as_param_dict(warm, attr: str) -> Optional[Dict[str, torch.Tensor]]:
    """A warm start given as the reference's state object or as a plain dict."""
    if warm is None:
        return None
    return getattr(warm, attr, warm)


def _certificate_record(value: torch.Tensor) -> Dict[str, Any]:
    return {"type": "convex_combo_max_negative", "max_value": float(value[0].item())}


@dataclass
class AlphaBetaStats:
    """Run statistics.  The branching decision stays on the device
    (``branch_layer`` / ``branch_neuron``, layer -1 = no ambiguous neuron);
    ``branch_choices`` converts it to the reference's list of
    ``(relu_input, index)`` on first access, so a run issues no host
    synchronization unless the caller asks for it."""

    feasibility: str = "unknown"
    reason: str = "ok"
    infeasible: Optional[torch.Tensor] = None
    # set when the first-layer certificate closed the query: {"type", "max_value"} as the
    # reference reports (alpha_beta_crown.py:484-531; its weights and halfspaces stay on the device)
    infeasible_certificate: Optional[Dict[str, Any]] = None
    steps: int = 0
    lr: float = 0.0
    branch_layer: Optional[torch.Tensor] = None
    branch_neuron: Optional[torch.Tensor] = None
    relu_names: Tuple[str, ...] = ()

    @property
    def branch_choices(self) -> Optional[List[Optional[Tuple[str, int]]]]:
        if self.branch_layer is None:
            return None
        lay = self.branch_layer.cpu().tolist()
        ids = self.branch_neuron.cpu().tolist()
        return [None if lay[i] < 0 else (self.relu_names[lay[i]], int(ids[i])) for i in range(len(lay))]


# Parameters of at most this many elements in all take the best-of copy inside the Adam step's
# launch (C4: 0.2 M elements, one launch fewer per step); larger ones keep the float4 copy kernel,
# which moves them faster than the step's per-element copy (C5's 8.4 M: 45.8 + 14.8 us apart,
# 67.8 us fused).
FUSED_COPY_MAX_ELEMS = 1 << 20


class _AdamGroup:
    """Device-resident Adam state of several parameter tensors, stepped together in
    one launch (the reference runs one torch.optim.Adam over every alpha and beta,
    alpha_beta_crown.py:747); each tensor has its own clamp after the step."""

    def __init__(self, params: List[torch.Tensor], clamps: List[Tuple[float, Optional[float]]]):
        self.p = params
        # the first step starts the moments at zero without reading them
        self.m = [torch.empty_like(t) for t in params]
        self.v = [torch.empty_like(t) for t in params]
        self.t = 0
        self.args = (_lib.ptr_array(self.p), _lib.ptr_array(self.m), _lib.ptr_array(self.v))
        self.n = _lib.i64_array([t.numel() for t in params])
        self.lo = _lib.f32_array([lo for lo, _hi in clamps])
        self.hi = _lib.f32_array([0.0 if hi is None else hi for _lo, hi in clamps])
        self.has_hi = _lib.i32_array([0 if hi is None else 1 for _lo, hi in clamps])

    def step(self, grads: List[torch.Tensor], lr: float, stream, best=None, improved=None, rows: int = 0) -> None:
        """One step; with ``best`` (one tensor per parameter) the rows flagged in ``improved``
        are first copied to it from the values the step updates (the best-of copy)."""
        self.t += 1
        _lib.call("bf_adam_clamp_multi", len(self.p), *self.args, _lib.ptr_array(grads), self.n, self.lo, self.hi,
                  self.has_hi, float(lr), 0.9, 0.999, 1e-8, self.t,
                  None if best is None else _lib.ptr_array(best), _lib.ptr(improved), int(rows), stream)


def branch_choices(trace: ForwardTrace, batch: int) -> List[Optional[Tuple[str, int]]]:
    """Widest ambiguous neuron per domain (alpha_beta_crown.py:145-182), on the device."""
    dev = next(iter(trace.relu_pre.values())).lower.device if trace.relu_pre else torch.device("cuda")
    gap = torch.full((batch,), float("-inf"), device=dev)
    layer = torch.full((batch,), -1, dtype=torch.int32, device=dev)
    idx = torch.zeros(batch, dtype=torch.int32, device=dev)
    names = list(trace.relu_pre.keys())
    stream = _lib.stream_handle()
    for li, name in enumerate(names):
        pre = trace.relu_pre[name]
        n = int(pre.lower[0].numel())
        _lib.call("bf_branch_update", _lib.ptr(pre.lower.reshape(batch, n)), _lib.ptr(pre.upper.reshape(batch, n)),
                  batch, n, li, _lib.ptr(gap), _lib.ptr(layer), _lib.ptr(idx), stream)
    lay = layer.cpu().tolist()
    ids = idx.cpu().tolist()
    return [None if lay[i] < 0 else (names[lay[i]], int(ids[i])) for i in range(batch)]


def branch_tensors(trace: ForwardTrace, batch: int):
    """Device tensors (layer index, neuron index, gap) of the branching rule."""
    dev = next(iter(trace.relu_pre.values())).lower.device
    gap = torch.full((batch,), float("-inf"), device=dev)
    layer = torch.full((batch,), -1, dtype=torch.int32, device=dev)
    idx = torch.zeros(batch, dtype=torch.int32, device=dev)
    stream = _lib.stream_handle()
    for li, (name, pre) in enumerate(trace.relu_pre.items()):
        n = int(pre.lower[0].numel())
        _lib.call("bf_branch_update", _lib.ptr(pre.lower.reshape(batch, n)), _lib.ptr(pre.upper.reshape(batch, n)),
                  batch, n, li, _lib.ptr(gap), _lib.ptr(layer), _lib.ptr(idx), stream)
    return layer, idx, gap


def alpha_from_crown(trace: ForwardTrace) -> Dict[str, torch.Tensor]:
    """Adaptive lower-slope init (native_alpha_beta_optimizer_schedule.py:635-653)."""
    out = {}
    stream = _lib.stream_handle()
    for name, pre in trace.relu_pre.items():
        a = torch.empty_like(pre.lower)
        _lib.call("bf_alpha_from_crown", _lib.ptr(pre.lower), _lib.ptr(pre.upper), pre.lower.numel(), _lib.ptr(a),
                  stream)
        out[name] = a
    return out


def _grad_pass(spec: InputSpec, chain: Chain, trace: ForwardTrace, saved: dict, B: int, S: int,
               alpha: Dict[str, Tuple[torch.Tensor, int]], splits: Dict[str, Tuple[torch.Tensor, int]],
               G: torch.Tensor) -> Tuple[Dict[str, torch.Tensor], Dict[str, torch.Tensor]]:
    """Reverse pass of the lower bound; returns dL/dalpha and dL/dbeta per ReLU ([B, n])."""
    dev = spec.center.device
    stream = _lib.stream_handle()
    layers = chain.layers
    M = B * S
    g = saved["h"]                       # dL/d(input coefficient)  [M, n_in0]
    cvec = saved["cvec"]                 # first-layer center projection [B, n_out0]
    g_alpha: Dict[str, torch.Tensor] = {}
    g_beta: Dict[str, torch.Tensor] = {}
    for k in range(0, len(layers) - 1):
        layer = layers[k]
        n_out = _numel(layer.out_shape)
        n_in = _numel(layer.in_shape)
        # rank-1 term: every row's bias contribution b += A~ . bias_k (and the center term on the input layer)
        if k == 0:
            vec = cvec if layer.bias is None else call_memo(saved, "cvec_bias", lambda: cvec + _bias_map(layer))
            vec_ld = n_out
        else:
            vec = _bias_map(layer) if layer.bias is not None else None
            vec_ld = 0
        gt = torch.empty(M, n_out, device=dev)
        if layer.kind == "linear":
            wsz = int(_lib.load().bf_gemm_rank1_workspace(M, n_out, n_in))
            ws = torch.empty(wsz, device=dev) if wsz else None
            with _timed("grad_gemm", 2.0 * M * n_in * n_out, 4.0 * (M * n_in + M * n_out + n_in * n_out)):
                _lib.call("bf_gemm_rank1", _lib.ptr(g), n_in, _lib.ptr(layer.weight.contiguous()), n_in, 1,
                          _lib.ptr(gt), n_out, M, n_out, n_in, S, _lib.ptr(G if vec is not None else None),
                          _lib.ptr(vec), vec_ld, _lib.ptr(ws), wsz, stream)
        else:
            Ci, Hi, Wi = layer.in_shape
            Co, Ho, Wo = layer.out_shape
            KH, KW = int(layer.weight.shape[2]), int(layer.weight.shape[3])
            sh, sw = layer.attrs["stride"]
            ph, pw = layer.attrs["padding"]
            with _timed("grad_conv", 2.0 * M * n_out * Ci * KH * KW, 4.0 * (M * n_in + M * n_out)):
                _lib.call("bf_conv2d_rows", _lib.ptr(g), 1, M, Ci, Hi, Wi, _lib.ptr(layer.weight.contiguous()), 0,
                          Co, KH, KW, sh, sw, ph, pw, Ho, Wo, _lib.ptr(gt), _lib.ptr(G if vec is not None else None),
                          _lib.ptr(vec), S if vec_ld else 1, vec_ld, stream)
        # through the ReLU relaxation of layer k's output
        name = layer.out_name
        pre = trace.relu_pre[name]
        A_in, a_stride = saved["A_in"][k]
        ga = torch.empty(B, n_out, device=dev)
        gb = torch.empty(B, n_out, device=dev)
        a_t, a_ld = alpha.get(name, (None, 0))
        sp, sp_ld = splits.get(name, (None, 0))
        g_in = torch.empty(M, n_out, device=dev)
        with _timed("relu_grad", 0.0, 4.0 * (3 * M * n_out + 4 * B * n_out)):
            _lib.call("bf_relu_grad", _lib.ptr(gt), _lib.ptr(A_in), a_stride, B, S, n_out,
                      _lib.ptr(pre.lower.reshape(B, n_out)), _lib.ptr(pre.upper.reshape(B, n_out)), _lib.ptr(a_t),
                      a_ld, _lib.ptr(G), _lib.ptr(sp), sp_ld, _lib.ptr(g_in), _lib.ptr(ga), _lib.ptr(gb), stream)
        g_alpha[name] = ga
        g_beta[name] = gb
        g = g_in
    return g_alpha, g_beta


def _evaluator(module, spec: InputSpec, trace, chain: Optional[Chain], linear_spec_C):
    """(bound, grad, out_dim) of the task: the chain's fused CROWN backward and its
    reverse pass, or the DAG backward of ``crown_dag`` and its reverse pass.
    bound(alpha, add, need_upper, need_lower, save) -> IntervalState;
    grad(saved, B, S, alpha_args, splits, G) -> (dL/dalpha, dL/dbeta)."""
    if chain is not None:
        def bound(alpha, add, need_upper, need_lower, save):
            return crown_backward(module, spec, trace, chain=chain, linear_spec_C=linear_spec_C, relu_alpha=alpha,
                                  relu_pre_add_coeff_l=add, need_upper=need_upper, need_lower=need_lower, save=save)

        def grad(saved, B, S, a_arg, splits, G):
            return _grad_pass(spec, chain, trace, saved, B, S, a_arg, splits, G)

        return bound, grad, _numel(chain.layers[-1].out_shape)
    from . import crown_dag

    def bound(alpha, add, need_upper, need_lower, save):
        return crown_dag.crown_backward_dag(module, spec, trace, linear_spec_C=linear_spec_C, relu_alpha=alpha,
                                            relu_pre_add_coeff_l=add, need_upper=need_upper, need_lower=need_lower,
                                            save=save)

    def grad(saved, B, S, a_arg, splits, G):
        return crown_dag.lower_grad_pass(module, spec, trace, saved, B, a_arg, splits, G)

    return bound, grad, _numel(trace.shapes[module.get_entry_task().output_values[0]])


def _relu_shapes(module, spec, chain: Optional[Chain]) -> Dict[str, Tuple[int, ...]]:
    """Per-sample shape of every ReLU input (op order), for a chain or a DAG task."""
    if chain is not None:
        return dict(chain.relu_shapes)
    from .crown_dag import relu_input_shapes
    return relu_input_shapes(module, spec)


def _chain_or_none(module, spec) -> Optional[Chain]:
    try:
        return parse_chain(module, spec)
    except NotAChain:
        return None


def _bias_map(layer) -> torch.Tensor:
    if layer.kind == "linear":
        return layer.bias.contiguous()
    Co, Ho, Wo = layer.out_shape
    return derived(f"conv_bias_map:{Ho}x{Wo}", (layer.bias,),
                   lambda: layer.bias.reshape(Co, 1).expand(Co, Ho * Wo).reshape(-1).contiguous())


def run_alpha_beta_crown_mlp(
    module,
    input_spec,
    *,
    linear_spec_C: Optional[torch.Tensor] = None,
    relu_split_state: Optional[Dict[str, torch.Tensor]] = None,
    steps: int = 20,
    lr: float = 0.2,
    alpha_init: float = 0.5,
    beta_init: float = 0.0,
    warm_start_alpha: Optional[Dict[str, torch.Tensor]] = None,
    warm_start_beta: Optional[Dict[str, torch.Tensor]] = None,
    objective: str = "lower",
    spec_reduce: str = "mean",
    per_batch_params: bool = False,
    trace: Optional[ForwardTrace] = None,
    raise_on_infeasible: bool = True,
    use_beta: bool = True,
    first_layer_certificate: bool = True,
    soft_tau: float = 1.0,
    lb_weight: float = 1.0,
    ub_weight: float = 1.0,
    record: Optional[list] = None,
):
    """HIP counterpart of run_alpha_beta_crown_mlp (alpha_beta_crown.py:643-941).

    ``use_beta=False`` drops the split multipliers (alpha-CROWN with splits
    applied only to the pre-activation boxes and relaxations,
    alpha_crown.py:137-261).  Returns (best_bounds, best_alpha, best_beta, stats).

    A single domain with a nonzero split is first checked by the first-layer
    split certificate (alpha_beta_crown.py:694-714); when it proves the splits
    infeasible the bounds are zeros of shape [1, 1], the parameter dicts are
    empty and ``stats.feasibility`` is "infeasible", as in the reference.  That
    check reads its verdict back to the host; callers that decide it
    themselves (the BaB rounds) pass ``first_layer_certificate=False``."""
    if objective not in _OBJECTIVES:
        raise AssertionError(f"unreachable objective: {objective}")
    if spec_reduce not in _REDUCTIONS:
        raise AssertionError(f"unreachable spec_reduce: {spec_reduce}")
    if spec_reduce == "softmin" and float(soft_tau) <= 0.0:
        raise ValueError(f"soft_tau must be >0, got {soft_tau}")
    spec = normalize_input_spec(input_spec)
    chain = _chain_or_none(module, spec)
    if (first_layer_certificate and relu_split_state and int(spec.center.shape[0]) == 1
            and any(bool((v != 0).any().item()) for v in relu_split_state.values() if v is not None)):
        from .split_certificate import check_flags, split_certificate
        shapes0 = _relu_shapes(module, spec, chain)
        value = torch.empty(1, device=spec.center.device, dtype=torch.float32)
        flag = split_certificate(module, spec, relu_split_state, shapes0, max_out=value).cpu().tolist()
        check_flags(flag)
        if flag[0] == 1:
            zeros = torch.zeros((1, 1), device=spec.center.device, dtype=torch.float32)
            return (IntervalState(lower=zeros, upper=zeros.clone()), AlphaState(), BetaState(),
                    AlphaBetaStats(feasibility="infeasible", reason="infeasible: first-layer split certificate",
                                   steps=int(steps), lr=float(lr),
                                   infeasible_certificate=_certificate_record(value)))
    if trace is None:
        trace = forward_ibp_trace(module, spec, relu_split_state=relu_split_state, chain=chain,
                                  raise_on_infeasible=raise_on_infeasible, relu_inputs_only=True)
    bound, grad, out_dim = _evaluator(module, spec, trace, chain, linear_spec_C)
    dev = spec.center.device
    B = int(spec.center.shape[0])
    stream = _lib.stream_handle()
    names = list(trace.relu_pre.keys())
    shapes = {n: tuple(int(d) for d in trace.relu_pre[n].lower.shape[1:]) for n in names}
    numel = {n: _numel(shapes[n]) for n in names}

    def init_param(warm, value):
        out = {}
        for n in names:
            target = (B, numel[n]) if per_batch_params else (numel[n],)
            if warm is not None and n in warm:
                t = warm[n].to(device=dev, dtype=torch.float32)
                if t.numel() == numel[n] and per_batch_params:
                    t = t.reshape(1, numel[n]).expand(B, numel[n])
                out[n] = t.reshape(target).contiguous().clone()
            else:
                out[n] = torch.full(target, float(value), device=dev, dtype=torch.float32)
        return out

    alpha = init_param(_as_param_dict(warm_start_alpha, "alpha_by_relu_input"), alpha_init)
    beta = init_param(_as_param_dict(warm_start_beta, "beta_by_relu_input"), beta_init)
    p_ld = {n: (numel[n] if per_batch_params else 0) for n in names}
    splits: Dict[str, Tuple[torch.Tensor, int]] = {}
    if relu_split_state:
        for n in names:
            if n in relu_split_state:
                s, ld = _broadcast_split(relu_split_state[n].to(dev), B, numel[n])
                splits[n] = (s, ld)
    # Every ReLU with a split state gets the split term.  The reference keeps those with a
    # nonzero entry (alpha_beta_crown.py:630-633); an all-zero split adds exact zeros and
    # receives a zero beta gradient (Adam then leaves beta unchanged), so the results are
    # the same, and no host synchronization is needed: the batch can be captured as a graph.
    beta_names = list(splits.keys()) if use_beta else []
    b_layer, b_neuron, _gap = branch_tensors(trace, B) if trace.relu_pre else (None, None, None)
    S = int(linear_spec_C.shape[-2]) if linear_spec_C is not None else out_dim
    M = B * S
    if objective != "lower" or spec_reduce != "mean":
        if record is not None:
            raise NotImplementedError("record is kept for the lower-bound objective with the mean reduction")
        best_lb, best_ub, best_alpha, best_beta = _optimise_general(
            module, spec, trace, chain, linear_spec_C, bound, grad, out_dim, B=B, S=S, names=names, numel=numel,
            alpha=alpha, beta=beta, p_ld=p_ld, splits=splits, beta_names=beta_names if objective == "lower" else [],
            steps=int(steps), lr=float(lr), objective=objective, spec_reduce=spec_reduce, soft_tau=float(soft_tau),
            lb_weight=float(lb_weight), ub_weight=float(ub_weight), per_batch_params=per_batch_params)
        out_alpha = AlphaState({n: best_alpha[n].reshape(((B,) if per_batch_params else ()) + shapes[n])
                                for n in names})
        out_beta = BetaState({n: best_beta[n].reshape(((B,) if per_batch_params else ()) + shapes[n]) for n in names})
        stats = AlphaBetaStats(infeasible=trace.infeasible, steps=int(steps), lr=float(lr), branch_layer=b_layer,
                               branch_neuron=b_neuron, relu_names=tuple(trace.relu_pre.keys()))
        return IntervalState(lower=best_lb, upper=best_ub), out_alpha, out_beta, stats
    # d(-sum_d mean_s lb)/dlb = -1/S ; d(-mean_d mean_s lb)/dlb = (-1/B)/S   (fp32, as autograd divides)
    g_row = np.float32(-1.0) / np.float32(S) if per_batch_params else (np.float32(-1.0) / np.float32(B)) / np.float32(S)
    G = torch.full((M,), float(g_row), device=dev, dtype=torch.float32)
    # one optimizer over every alpha (clamped to [0, 1]) and every split multiplier (>= 0)
    adam = _AdamGroup([alpha[n] for n in names] + [beta[n] for n in beta_names],
                      [(0.0, 1.0)] * len(names) + [(0.0, None)] * len(beta_names))
    best_metric = torch.empty(B, device=dev)
    best_lb = torch.empty(B, S, device=dev)
    improved = torch.empty(B, dtype=torch.int32, device=dev)
    best_alpha = {n: alpha[n].clone() for n in names}
    best_beta = {n: beta[n].clone() for n in names}
    best_scalar = None
    add = {n: torch.empty(B, numel[n], device=dev) for n in beta_names}
    beta_args = (_lib.ptr_array([beta[n] for n in beta_names]), _lib.i64_array([p_ld[n] for n in beta_names]),
                 _lib.ptr_array([splits[n][0] for n in beta_names]), _lib.i64_array([splits[n][1] for n in beta_names]),
                 _lib.i64_array([numel[n] for n in beta_names]), B, _lib.ptr_array([add[n] for n in beta_names]))
    # the best-of copy: alpha of every ReLU, beta of those that move (the others keep their initial value)
    copy_dst = [best_alpha[n] for n in names] + [best_beta[n] for n in beta_names]
    copy_args = (_lib.ptr_array(copy_dst), _lib.ptr_array([alpha[n] for n in names] + [beta[n] for n in beta_names]),
                 _lib.i64_array([numel[n] for n in names] + [numel[n] for n in beta_names]), B, _lib.ptr(improved))
    memo: dict = {}   # per-call operands (scaled gradient rows, center-plus-bias), freed with the call
    fuse_copy = per_batch_params and sum(int(t.numel()) for t in adam.p) <= FUSED_COPY_MAX_ELEMS
    for step in range(int(steps) + 1):
        if beta_names:
            _lib.call("bf_beta_coeff_multi", len(beta_names), *beta_args, stream)
        saved = {"grad_rows": G, "memo": memo} if step < int(steps) else None
        # lower bound only: the objective and the best-of rule read nothing else
        bounds = bound({n: alpha[n] for n in names}, {n: add[n] for n in beta_names}, False, True, saved)
        if per_batch_params:
            _lib.call("bf_best_update", _lib.ptr(bounds.lower), None, B, S, _lib.ptr(best_metric),
                      _lib.ptr(best_lb), None, _lib.ptr(improved), 1 if step == 0 else 0, stream)
            if not fuse_copy or step == int(steps):
                # a launch of its own: large parameters (the float4 copy kernel moves them faster than
                # the step's per-element copy), or the last evaluation (no step follows)
                _lib.call("bf_masked_copy_rows_multi", len(copy_dst), *copy_args, stream)
        else:
            metric = float(bounds.lower.mean().item())
            if best_scalar is None or metric > best_scalar:
                best_scalar = metric
                best_lb.copy_(bounds.lower)
                for n in names:
                    best_alpha[n].copy_(alpha[n])
                    best_beta[n].copy_(beta[n])
        if record is not None:
            pshape = {n: ((B,) if per_batch_params else ()) + shapes[n] for n in names}
            record.append({"step": step, "alpha": {n: alpha[n].reshape(pshape[n]).cpu() for n in names},
                           "beta": {n: beta[n].reshape(pshape[n]).cpu() for n in names},
                           "lower": bounds.lower.cpu()})
        if step == int(steps):
            break
        a_arg = {n: (alpha[n], p_ld[n]) for n in names}
        g_alpha, g_beta = grad(saved, B, S, a_arg, splits, G)
        if not per_batch_params:
            for d in (g_alpha, g_beta):
                for n in names:
                    r = torch.empty(numel[n], device=dev)
                    _lib.call("bf_sum_rows", _lib.ptr(d[n]), B, numel[n], _lib.ptr(r), stream)
                    d[n] = r
        # small parameters: the step takes the best-of copy of this evaluation's parameters with it
        # (rows = domains), one launch fewer per step
        adam.step([g_alpha[n] for n in names] + [g_beta[n] for n in beta_names], lr, stream,
                  best=copy_dst if fuse_copy else None, improved=improved, rows=B)
        if record is not None:
            rec = record[-1]
            rec["grad_alpha"] = {n: g_alpha[n].reshape(pshape[n]).cpu() for n in names}
            rec["grad_beta"] = {n: (g_beta[n].reshape(pshape[n]).cpu() if n in beta_names else None) for n in names}
            rec["alpha_next"] = {n: alpha[n].reshape(pshape[n]).cpu() for n in names}
            rec["beta_next"] = {n: beta[n].reshape(pshape[n]).cpu() for n in names}
    # The reference keeps the upper bound of the evaluation that gave the best lower
    # bound.  The upper bound depends on alpha alone (beta enters the lower bound
    # only) and every domain's rows on that domain's parameters alone, so one upper
    # pass with the best parameters reproduces it.
    best_ub = bound({n: best_alpha[n] for n in names}, None, True, False, None).upper
    out_alpha = AlphaState({n: best_alpha[n].reshape(((B,) if per_batch_params else ()) + shapes[n]) for n in names})
    out_beta = BetaState({n: best_beta[n].reshape(((B,) if per_batch_params else ()) + shapes[n]) for n in names})
    stats = AlphaBetaStats(infeasible=trace.infeasible, steps=int(steps), lr=float(lr), branch_layer=b_layer,
                           branch_neuron=b_neuron, relu_names=tuple(trace.relu_pre.keys()))
    return IntervalState(lower=best_lb, upper=best_ub), out_alpha, out_beta, stats


_OBJECTIVES = {"lower": 0, "upper": 1, "gap": 2, "both": 3}
_REDUCTIONS = {"mean": 0, "min": 1, "softmin": 2}


def _optimise_general(module, spec, trace, chain, linear_spec_C, bound, grad, out_dim, *, B, S, names, numel,
                      alpha, beta, p_ld, splits, beta_names, steps, lr, objective, spec_reduce, soft_tau, lb_weight,
                      ub_weight, per_batch_params):
    """The optimisation loop for every objective and spec reduction but ("lower",
    "mean") (alpha_beta_crown.py:756-815).  The upper bound of C is computed as
    minus the lower bound of -C, the same arithmetic with every term negated
    (exactly), so one lower-bound pass and its reverse pass serve both bounds.
    Per step ``bf_objective_step`` reduces the bounds to each domain's metric,
    gives the loss's row gradients and updates the best-of state; the
    concretization seeds are formed with unit row weights and scaled by the row
    gradients after the pass (the same products, rounded once).  Objectives other
    than "lower" leave the split multipliers out of the bound (and unchanged).
    Returns (best lower, best upper, best alpha, best beta)."""
    dev = spec.center.device
    stream = _lib.stream_handle()
    M = B * S
    obj = _OBJECTIVES[objective]
    use_l = objective in ("lower", "gap", "both")
    use_u = objective in ("upper", "gap", "both")
    C = linear_spec_C
    if C is None:
        C = torch.eye(out_dim, device=dev).unsqueeze(0).expand(B, out_dim, out_dim)
    C_neg = (-C).contiguous()
    bound_u, grad_u, _ = _evaluator(module, spec, trace, chain, C_neg)
    ones = torch.ones(M, device=dev)
    g_scale = float(np.float32(-1.0)) if per_batch_params else float(np.float32(-1.0) / np.float32(B))
    G_l = torch.empty(M, device=dev) if use_l else None
    G_nu = torch.empty(M, device=dev) if use_u else None
    metric = torch.empty(B, device=dev)
    best_metric = torch.empty(B, device=dev)
    best_lb = torch.empty(B, S, device=dev)
    best_ub = torch.empty(B, S, device=dev)
    improved = torch.empty(B, dtype=torch.int32, device=dev)
    best_scalar = None
    adam = _AdamGroup([alpha[n] for n in names] + [beta[n] for n in beta_names],
                      [(0.0, 1.0)] * len(names) + [(0.0, None)] * len(beta_names))
    best_alpha = {n: alpha[n].clone() for n in names}
    best_beta = {n: beta[n].clone() for n in names}
    add = {n: torch.empty(B, numel[n], device=dev) for n in beta_names}
    beta_args = (_lib.ptr_array([beta[n] for n in beta_names]), _lib.i64_array([p_ld[n] for n in beta_names]),
                 _lib.ptr_array([splits[n][0] for n in beta_names]), _lib.i64_array([splits[n][1] for n in beta_names]),
                 _lib.i64_array([numel[n] for n in beta_names]), B, _lib.ptr_array([add[n] for n in beta_names]))
    copy_dst = [best_alpha[n] for n in names] + [best_beta[n] for n in beta_names]
    copy_args = (_lib.ptr_array(copy_dst), _lib.ptr_array([alpha[n] for n in names] + [beta[n] for n in beta_names]),
                 _lib.i64_array([numel[n] for n in names] + [numel[n] for n in beta_names]), B, _lib.ptr(improved))
    memo_l: dict = {}
    memo_u: dict = {}
    for step in range(steps + 1):
        last = step == steps
        if beta_names:
            _lib.call("bf_beta_coeff_multi", len(beta_names), *beta_args, stream)
        cur = {n: alpha[n] for n in names}
        saved_l = {"grad_rows": ones, "memo": memo_l} if (use_l and not last) else None
        saved_u = {"grad_rows": ones, "memo": memo_u} if (use_u and not last) else None
        lb = bound(cur, {n: add[n] for n in beta_names}, False, True, saved_l).lower if use_l else None
        nub = bound_u(cur, None, False, True, saved_u).lower if use_u else None
        if per_batch_params:
            _lib.call("bf_objective_step", _lib.ptr(lb), _lib.ptr(nub), B, S, obj, _REDUCTIONS[spec_reduce], soft_tau,
                      lb_weight, ub_weight, g_scale, _lib.ptr(metric), _lib.ptr(G_l), _lib.ptr(G_nu),
                      _lib.ptr(best_metric), _lib.ptr(best_lb if use_l else None),
                      _lib.ptr(best_ub if use_u else None), _lib.ptr(improved), 1 if step == 0 else 0, stream)
            _lib.call("bf_masked_copy_rows_multi", len(copy_dst), *copy_args, stream)
        else:
            _lib.call("bf_objective_step", _lib.ptr(lb), _lib.ptr(nub), B, S, obj, _REDUCTIONS[spec_reduce], soft_tau,
                      lb_weight, ub_weight, g_scale, _lib.ptr(metric), _lib.ptr(G_l), _lib.ptr(G_nu), None, None,
                      None, None, 0, stream)
            value = float(metric.mean().item())   # the reference compares metric_b.mean() as a Python float
            if best_scalar is None or value > best_scalar:
                best_scalar = value
                if use_l:
                    best_lb.copy_(lb)
                if use_u:
                    torch.neg(nub, out=best_ub)
                for n in names:
                    best_alpha[n].copy_(alpha[n])
                    best_beta[n].copy_(beta[n])
        if last:
            break
        a_arg = {n: (alpha[n], p_ld[n]) for n in names}
        g_alpha: Dict[str, torch.Tensor] = {}
        g_beta: Dict[str, torch.Tensor] = {}
        for saved, gfun, Grow in ((saved_l, grad, G_l), (saved_u, grad_u, G_nu)):
            if saved is None:
                continue
            if "h" in saved:
                h = saved["h"]
                _lib.call("bf_scale_rows", _lib.ptr(h), M, int(h.numel() // M), _lib.ptr(Grow), stream)
            ga, gb = gfun(saved, B, S, a_arg, splits, Grow)
            for n in names:
                g_alpha[n] = ga[n] if n not in g_alpha else g_alpha[n] + ga[n]
                if n in beta_names:
                    g_beta[n] = gb[n] if n not in g_beta else g_beta[n] + gb[n]
        if not per_batch_params:
            for d in (g_alpha, g_beta):
                for n in list(d.keys()):
                    r = torch.empty(numel[n], device=dev)
                    _lib.call("bf_sum_rows", _lib.ptr(d[n]), B, numel[n], _lib.ptr(r), stream)
                    d[n] = r
        adam.step([g_alpha[n] for n in names] + [g_beta[n] for n in beta_names], lr, stream)
    # the bound the objective did not follow, at the best parameters (domains are
    # independent and, outside the "lower" objective, the multipliers do not enter it)
    if not use_l:
        best_lb = bound({n: best_alpha[n] for n in names}, None, False, True, None).lower
    if not use_u:
        best_ub = bound({n: best_alpha[n] for n in names}, None, True, False, None).upper
    return best_lb, best_ub, best_alpha, best_beta


def check_first_layer_infeasible_split(module, input_spec, *,
                                       relu_split_state: Dict[str, torch.Tensor]) -> AlphaBetaStats:
    """alpha_beta_crown.py:109-142: feasibility "infeasible" when the first-layer split
    certificate (``bf_split_certificate``: a convex combination of the split halfspaces
    whose maximum over the input set is below -1e-6) closes the one-input query, else
    "unknown" (also for batches of more than one input, which the reference skips)."""
    from .split_certificate import check_flags, split_certificate
    module.validate()
    spec = normalize_input_spec(input_spec)
    if int(spec.center.shape[0]) != 1:
        return AlphaBetaStats(feasibility="unknown", reason="skip (batch!=1)")
    if not relu_split_state or not any(bool((v != 0).any().item()) for v in relu_split_state.values()
                                       if v is not None):
        return AlphaBetaStats(feasibility="unknown", reason="ok (no first-layer split halfspaces)")
    value = torch.empty(1, device=spec.center.device, dtype=torch.float32)
    flag = split_certificate(module, spec, relu_split_state, _relu_shapes(module, spec, _chain_or_none(module, spec)),
                             max_out=value)
    flag = flag.cpu().tolist()
    check_flags(flag)
    if flag[0] == 1:
        return AlphaBetaStats(feasibility="infeasible", reason="infeasible: first-layer split certificate",
                              infeasible_certificate=_certificate_record(value))
    return AlphaBetaStats(feasibility="unknown", reason="ok")


def run_alpha_crown_mlp(module, input_spec, *, linear_spec_C=None, steps: int = 20, lr: float = 0.2,
                        alpha_init: float = 0.5, objective: str = "lower", spec_reduce: str = "mean",
                        soft_tau: float = 1.0, lb_weight: float = 1.0, ub_weight: float = 1.0,
                        warm_start: Optional[Dict[str, torch.Tensor]] = None,
                        relu_split_state=None, trace: Optional[ForwardTrace] = None):
    """HIP counterpart of run_alpha_crown_mlp (alpha_crown.py:137-261): alpha shared
    by all domains, no split multipliers, best-of on the batch mean of the
    objective's metric.  The reference reduces "mean" over every [B, S] element at
    once and the shared alpha-beta loop over specs and then domains: the same
    value up to summation order.  ``warm_start`` maps ReLU input names to alpha
    tensors of the ReLU's logical shape."""
    bounds, alpha, _beta, stats = run_alpha_beta_crown_mlp(
        module, input_spec, linear_spec_C=linear_spec_C, relu_split_state=relu_split_state, steps=steps, lr=lr,
        alpha_init=alpha_init, warm_start_alpha=warm_start, per_batch_params=False, use_beta=False, trace=trace,
        objective=objective, spec_reduce=spec_reduce, soft_tau=soft_tau, lb_weight=lb_weight, ub_weight=ub_weight,
        first_layer_certificate=False)   # alpha_crown.py has no certificate
    return bounds, alpha, stats


def run_alpha_crown_from_crown_init(module, input_spec, *, linear_spec_C=None, steps: int = 20, lr: float = 0.1,
                                    record: Optional[list] = None):
    """Config C4: per-domain alpha initialised from the CROWN relaxation
    (alpha_from_crown), then ``steps`` Adam steps on the lower bound."""
    spec = normalize_input_spec(input_spec)
    trace = forward_ibp_trace(module, spec, chain=_chain_or_none(module, spec), relu_inputs_only=True)
    init = alpha_from_crown(trace)
    return run_alpha_beta_crown_mlp(module, spec, linear_spec_C=linear_spec_C, steps=steps, lr=lr,
                                    warm_start_alpha=init, per_batch_params=True, trace=trace, record=record)


def lower_bound_gradients(module, input_spec, *, linear_spec_C, relu_alpha: Dict[str, torch.Tensor],
                          relu_beta: Optional[Dict[str, torch.Tensor]] = None,
                          relu_split_state: Optional[Dict[str, torch.Tensor]] = None, per_batch_params: bool = True):
    """One evaluation plus one reverse pass: returns (bounds, dL/dalpha, dL/dbeta)
    for L = -sum_d mean_s lb (per-domain parameters) or -mean lb (shared)."""
    spec = normalize_input_spec(input_spec)
    chain = _chain_or_none(module, spec)
    trace = forward_ibp_trace(module, spec, relu_split_state=relu_split_state, chain=chain, relu_inputs_only=True)
    bound, grad, _out_dim = _evaluator(module, spec, trace, chain, linear_spec_C)
    dev = spec.center.device
    B = int(spec.center.shape[0])
    names = list(trace.relu_pre.keys())
    numel = {n: int(trace.relu_pre[n].lower[0].numel()) for n in names}
    S = int(linear_spec_C.shape[-2])
    g_row = np.float32(-1.0) / np.float32(S) if per_batch_params else (np.float32(-1.0) / np.float32(B)) / np.float32(S)
    G = torch.full((B * S,), float(g_row), device=dev, dtype=torch.float32)
    stream = _lib.stream_handle()
    alpha = {n: relu_alpha[n].reshape((B, numel[n]) if per_batch_params else (numel[n],)).contiguous()
             for n in names}
    p_ld = {n: (numel[n] if per_batch_params else 0) for n in names}
    splits: Dict[str, Tuple[torch.Tensor, int]] = {}
    add = {}
    if relu_split_state:
        for n in names:
            if n in relu_split_state:
                splits[n] = _broadcast_split(relu_split_state[n].to(dev), B, numel[n])
                if relu_beta is not None and bool((splits[n][0] != 0).any().item()):
                    b = relu_beta[n].reshape((B, numel[n]) if per_batch_params else (numel[n],)).contiguous()
                    add[n] = torch.empty(B, numel[n], device=dev)
                    _lib.call("bf_beta_coeff", _lib.ptr(b), p_ld[n], _lib.ptr(splits[n][0]), splits[n][1], B,
                              numel[n], _lib.ptr(add[n]), stream)
    saved = {"grad_rows": G}
    # the chain's pass computes both bounds; the DAG pass follows the lower bound alone
    bounds = bound(alpha, add, chain is not None, True, saved)
    g_alpha, g_beta = grad(saved, B, S, {n: (alpha[n], p_ld[n]) for n in names}, splits, G)
    if not per_batch_params:
        for d in (g_alpha, g_beta):
            for n in list(d.keys()):
                r = torch.empty(numel[n], device=dev)
                _lib.call("bf_sum_rows", _lib.ptr(d[n]), B, numel[n], _lib.ptr(r), stream)
                d[n] = r
    return bounds, g_alpha, g_beta
