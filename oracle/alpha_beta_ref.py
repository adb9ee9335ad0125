"""CPU restatement of the reference alpha / alpha-beta CROWN optimisers and the
BaB node-batch evaluation (test infrastructure only).

* ``branch_choices`` -- boundflow/runtime/alpha_beta_crown.py:145-182
* ``beta_to_pre_add`` -- boundflow/runtime/alpha_beta_crown.py:615-640
* ``run_alpha_beta_crown`` -- boundflow/runtime/alpha_beta_crown.py:643-941, with
  the B==1 first-layer infeasibility pre-check of :694-714
* ``first_layer_split_halfspaces`` -- boundflow/runtime/alpha_beta_crown.py:259-389
* ``split_certificate`` -- ``_is_infeasible_split_first_layer_convex_combo``,
  boundflow/runtime/alpha_beta_crown.py:391-532
* ``run_alpha_crown`` -- boundflow/runtime/alpha_crown.py:137-261
* ``adaptive_alpha_init`` -- boundflow/runtime/native_alpha_beta_optimizer_schedule.py:635-653
* ``evaluate_domain_batch`` -- the node-batch section of boundflow/runtime/bab.py:1250-1460
  with the certification rule of boundflow/runtime/bab.py:870-895
"""

from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch

from boundflow_amd.ir import BFTaskModule
from boundflow_amd.spec import InputSpec, IntervalState, normalize_input_spec

from .crown_ref import (DenseOp, _pair, broadcast_split, concretize_affine, conv2d_right, crown_backward_from_trace,
                        forward_ibp_trace)


def branch_choices(relu_pre: Dict[str, IntervalState]) -> List[Optional[Tuple[str, int]]]:
    """alpha_beta_crown.py:145-182: widest ambiguous neuron per domain."""
    if not relu_pre:
        return []
    any_pre = next(iter(relu_pre.values()))
    bsz = int(any_pre.lower.shape[0])
    best_name: List[Optional[str]] = [None] * bsz
    best_idx = [0] * bsz
    best_gap = torch.full((bsz,), float("-inf"), dtype=any_pre.lower.dtype)
    for name, pre in relu_pre.items():
        l = pre.lower.reshape(int(pre.lower.shape[0]), -1)
        u = pre.upper.reshape(int(pre.upper.shape[0]), -1)
        amb = (l < 0) & (u > 0)
        if not amb.any():
            continue
        gap = (u - l).clamp_min(0.0)
        gap = torch.where(amb, gap, torch.full_like(gap, float("-inf")))
        row_best = gap.max(dim=1).values
        row_idx = gap.argmax(dim=1)
        improve = row_best > best_gap
        if improve.any():
            best_gap = torch.where(improve, row_best, best_gap)
            for i in improve.nonzero(as_tuple=False).flatten().tolist():
                best_name[i] = name
                best_idx[i] = int(row_idx[i].item())
    return [None if best_name[i] is None else (best_name[i], int(best_idx[i])) for i in range(bsz)]


def _flatten_param(value: torch.Tensor, pre: IntervalState) -> torch.Tensor:
    """alpha_beta_crown.py:63-110."""
    shape = tuple(int(d) for d in pre.lower.shape[1:])
    flat = 1
    for d in shape:
        flat *= d
    batch = int(pre.lower.shape[0])
    if value.dim() == 0:
        return value.reshape(1, 1).expand(batch, flat)
    if tuple(value.shape) == shape or (value.dim() == 1 and int(value.shape[0]) == flat):
        return value.reshape(1, flat).expand(batch, flat)
    if int(value.shape[0]) == 1 and value.numel() == flat:
        return value.reshape(1, flat).expand(batch, flat)
    return value.reshape(batch, flat)


def beta_to_pre_add(beta: Dict[str, torch.Tensor], relu_pre, relu_split_state) -> Dict[str, torch.Tensor]:
    """alpha_beta_crown.py:615-640: add_l = -beta * s * 1[s != 0]."""
    if not relu_split_state:
        return {}
    out: Dict[str, torch.Tensor] = {}
    for name, b in beta.items():
        split = relu_split_state.get(name)
        pre = relu_pre.get(name)
        if split is None or pre is None:
            continue
        s_b = broadcast_split(split, pre.lower)
        beta_b = _flatten_param(b, pre)
        mask = s_b != 0
        if not mask.any():
            continue
        s_f = s_b.to(dtype=b.dtype)
        out[name] = -beta_b * s_f * mask.to(dtype=b.dtype)
    return out


def has_nonzero_split(relu_split_state) -> bool:
    """alpha_beta_crown.py:53-60."""
    return any(v is not None and v.numel() > 0 and bool((v != 0).any()) for v in (relu_split_state or {}).values())


def first_layer_split_halfspaces(module: BFTaskModule, spec: InputSpec, relu_split_state):
    """alpha_beta_crown.py:259-389: for every ReLU (op order) whose input is made by
    a linear or conv2d op reading the network input, one halfspace
    (name, neuron, a = s * row, c = s * bias) per nonzero split entry, in neuron
    order.  A conv row is the one-hot output neuron pulled back through the conv."""
    if not has_nonzero_split(relu_split_state):
        return []
    task = module.get_entry_task()
    params = module.params
    _env, relu_pre = forward_ibp_trace(module, spec)
    producer = {op.outputs[0]: op for op in task.ops if op.outputs}
    out = []
    for op in task.ops:
        if op.op_type != "relu":
            continue
        x = op.inputs[0]
        split = relu_split_state.get(x)
        if split is None or x not in relu_pre:
            continue
        flat = broadcast_split(split, relu_pre[x].lower)
        prod = producer.get(x)
        if prod is None or not prod.inputs or prod.inputs[0] != spec.value_name or int(flat.shape[0]) != 1:
            continue
        vec = flat[0]
        if prod.op_type == "linear":
            W = params.get(prod.inputs[1])
            if W is None or W.dim() != 2 or int(W.shape[0]) != int(vec.shape[0]):
                continue
            b = params.get(prod.inputs[2]) if len(prod.inputs) == 3 else torch.zeros(int(W.shape[0]), dtype=W.dtype)
            if b is None or b.dim() != 1 or int(b.shape[0]) != int(W.shape[0]):
                continue
            for i in range(int(vec.shape[0])):
                s = int(vec[i])
                if s != 0:
                    out.append((x, i, float(s) * W[i], float(s) * b[i]))
            continue
        if prod.op_type != "conv2d":
            continue
        W = params.get(prod.inputs[1])
        if W is None or W.dim() != 4 or spec.center.dim() != 4:
            continue
        oshape = tuple(int(d) for d in relu_pre[x].lower.shape[1:])
        if len(oshape) != 3:
            continue
        b = params.get(prod.inputs[2]) if len(prod.inputs) == 3 else None
        if b is None:
            b = torch.zeros(int(W.shape[0]), dtype=W.dtype)
        ishape = tuple(int(d) for d in spec.center.shape[1:])
        a = prod.attrs
        for fi in range(int(vec.shape[0])):
            s = int(vec[fi])
            if s == 0:
                continue
            one_hot = torch.zeros((1, 1) + oshape, dtype=W.dtype)
            one_hot.view(-1)[fi] = 1.0
            # the reference's conv2d_right pairs scalar attributes (linear_operator.py:434-436)
            row = conv2d_right(DenseOp(one_hot, oshape), W, _pair(a.get("stride", 1)), _pair(a.get("padding", 0)),
                               _pair(a.get("dilation", 1)), int(a.get("groups", 1)), ishape, oshape).to_dense()[0, 0]
            ch = fi // (oshape[1] * oshape[2])
            out.append((x, fi, float(s) * row.reshape(-1), float(s) * b[ch]))
    return out


def split_certificate(module: BFTaskModule, input_spec, relu_split_state, *, steps: int = 200, lr: float = 0.1,
                      tol: float = 1e-6, return_value: bool = False):
    """alpha_beta_crown.py:391-532: the first-layer split halfspaces have no common
    point in the input set when some convex combination of them has a maximum
    over the set below -tol.  One halfspace is checked directly; several by
    Adam on the softmax logits of the combination (from 0, ``steps`` steps,
    stopping at the first maximum below -tol).  ``return_value`` appends the
    certificate's max_value (the maximum that closed the node, as the reference's
    certificate record holds it), or None when the node is not closed."""
    spec = normalize_input_spec(input_spec)
    hs = first_layer_split_halfspaces(module, spec, relu_split_state)
    if not hs:
        return (False, "ok (no first-layer split halfspaces)", None) if return_value else (
            False, "ok (no first-layer split halfspaces)")
    if int(spec.center.shape[0]) != 1:
        return (False, "skip (batch!=1)", None) if return_value else (False, "skip (batch!=1)")
    dtype = spec.center.dtype
    ishape = tuple(int(d) for d in spec.center.shape[1:])
    a_mat = torch.stack([h[2].to(dtype) for h in hs], dim=0).detach()
    c_vec = torch.stack([h[3].to(dtype) for h in hs], dim=0).detach()

    def upper(a, c):
        _lb, ub = concretize_affine(spec, spec.center, DenseOp(a.view(1, 1, -1), ishape), c.view(1, 1))
        return ub.squeeze()

    def out(flag, reason, value=None):
        return (flag, reason, value) if return_value else (flag, reason)

    if len(hs) == 1:
        ub0 = float(upper(a_mat[0], c_vec[0]).item())
        return out(True, "infeasible: single halfspace", ub0) if ub0 < -float(tol) else out(False, "ok")
    logits = torch.zeros(len(hs), dtype=dtype, requires_grad=True)
    opt = torch.optim.Adam([logits], lr=float(lr))
    for _ in range(int(steps)):
        w = torch.softmax(logits, dim=0)
        ub0 = upper((w.unsqueeze(1) * a_mat).sum(dim=0), (w * c_vec).sum())
        val = float(ub0.detach().item())
        if val < -float(tol):
            return out(True, "infeasible: convex combination", val)
        opt.zero_grad(set_to_none=True)
        ub0.backward()
        opt.step()
    return out(False, "ok")


def adaptive_alpha_init(relu_pre: Dict[str, IntervalState]) -> Dict[str, torch.Tensor]:
    """native_alpha_beta_optimizer_schedule.py:635-653 ("from CROWN" slope init)."""
    out = {}
    for name, value in relu_pre.items():
        positive = value.lower >= 0
        negative = value.upper <= 0
        ambiguous = ~(positive | negative)
        alpha = torch.zeros_like(value.lower)
        alpha[positive] = 1.0
        alpha[ambiguous] = (value.upper[ambiguous] > -value.lower[ambiguous]).to(dtype=value.lower.dtype)
        out[name] = alpha
    return out


def run_alpha_beta_crown(
    module: BFTaskModule,
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
    per_batch_params: bool = False,
    forward_trace=None,
    return_feasibility: bool = False,
    record: Optional[list] = None,
    objective: str = "lower",
    spec_reduce: str = "mean",
    soft_tau: float = 1.0,
    lb_weight: float = 1.0,
    ub_weight: float = 1.0,
):
    """alpha_beta_crown.py:643-941.  ``objective`` "lower" maximises the reduced lower
    bound with the split multipliers in the bound; "upper", "gap" and "both" use
    the bounds without them (alpha_beta_crown.py:756-785) and the metrics
    -R_max(ub), -R_max(ub - lb) and lb_weight R_min(lb) - ub_weight R_max(ub); the
    spec reduction R is the mean, min / max, or softmin / softmax with temperature
    ``soft_tau`` (:787-815).

    Returns (best_bounds, best_alpha, best_beta, branch_choices), plus the
    feasibility ("infeasible" or "unknown") with ``return_feasibility``.  A
    single domain with splits is first checked by ``split_certificate``
    (:694-714); when it proves the splits infeasible the bounds are zeros of
    shape [1, 1], the parameter dicts empty and the branch choices None.

    ``record`` (a list) receives one dict per evaluation: the parameters it used
    (``alpha``, ``beta``), its bounds, and for the steps that update them the
    gradients, Adam's moments before the update (``exp_avg``, ``exp_avg_sq``;
    zeros before the first) and the clamped parameters after it (``alpha_next``,
    ``beta_next``) -- the state the per-step parity tests feed to the device.
    """
    module.validate()
    spec = normalize_input_spec(input_spec)
    dtype = spec.center.dtype
    batch = int(spec.center.shape[0])
    if batch == 1 and has_nonzero_split(relu_split_state or {}):
        infeasible, _reason = split_certificate(module, spec, relu_split_state)
        if infeasible:
            zeros = torch.zeros((1, 1), dtype=dtype)
            out = (IntervalState(zeros, zeros.clone()), {}, {}, None)
            return out + ("infeasible",) if return_feasibility else out
    if forward_trace is None:
        interval_env, relu_pre = forward_ibp_trace(module, spec, relu_split_state=relu_split_state)
    else:
        interval_env, relu_pre = forward_trace
    shapes = {name: tuple(int(d) for d in pre.lower.shape[1:]) for name, pre in relu_pre.items()}

    def _init(warm, init_value):
        out = {}
        for name, shape in shapes.items():
            target = ((batch,) + shape) if per_batch_params else shape
            if warm is not None and name in warm:
                out[name] = warm[name].to(dtype=dtype).reshape(target).detach().clone()
            else:
                out[name] = torch.full(target, float(init_value), dtype=dtype)
        return out

    alpha = {k: v.requires_grad_(True) for k, v in _init(warm_start_alpha, alpha_init).items()}
    beta = {k: v.requires_grad_(True) for k, v in _init(warm_start_beta, beta_init).items()}
    params = list(alpha.values()) + list(beta.values())
    opt = torch.optim.Adam(params, lr=float(lr))

    best_metric = None
    best_metric_scalar = None
    best_bounds = None
    best_alpha = None
    best_beta = None
    choices = branch_choices(relu_pre)
    def reduce_specs(x, direction):
        if x.dim() != 2:
            return x.mean().expand(batch)
        if spec_reduce == "mean":
            return x.mean(dim=1)
        if spec_reduce == "min":
            return x.min(dim=1).values if direction == "min" else x.max(dim=1).values
        if spec_reduce == "softmin":
            tau = float(soft_tau)
            if tau <= 0.0:
                raise ValueError(f"soft_tau must be >0, got {soft_tau}")
            if direction == "min":
                return -tau * torch.logsumexp(-x / tau, dim=1)
            return tau * torch.logsumexp(x / tau, dim=1)
        raise AssertionError(f"unreachable spec_reduce: {spec_reduce}")

    for step in range(int(steps) + 1):
        add_l = beta_to_pre_add(beta, relu_pre, relu_split_state) if objective == "lower" else None
        bounds = crown_backward_from_trace(
            module, spec, interval_env=interval_env, relu_pre=relu_pre, linear_spec_C=linear_spec_C,
            relu_alpha=alpha, relu_pre_add_coeff_l=add_l,
        )
        if objective == "lower":
            metric_b = reduce_specs(bounds.lower, "min")
        elif objective == "upper":
            metric_b = -reduce_specs(bounds.upper, "max")
        elif objective == "gap":
            metric_b = -reduce_specs(bounds.upper - bounds.lower, "max")
        elif objective == "both":
            metric_b = float(lb_weight) * reduce_specs(bounds.lower, "min") - float(ub_weight) * reduce_specs(
                bounds.upper, "max")
        else:
            raise AssertionError(f"unreachable objective: {objective}")
        metric = metric_b.mean()
        if record is not None:
            record.append({"step": step, "alpha": {k: v.detach().clone() for k, v in alpha.items()},
                           "beta": {k: v.detach().clone() for k, v in beta.items()},
                           "lower": bounds.lower.detach().clone(), "upper": bounds.upper.detach().clone()})
        if best_metric is None:
            best_metric = metric_b.detach().clone()
            best_metric_scalar = metric.detach().clone()
            best_bounds = IntervalState(bounds.lower.detach().clone(), bounds.upper.detach().clone())
            best_alpha = {k: v.detach().clone() for k, v in alpha.items()}
            best_beta = {k: v.detach().clone() for k, v in beta.items()}
        else:
            if per_batch_params:
                improve = metric_b.detach() > best_metric
                if improve.any():
                    best_metric = torch.where(improve, metric_b.detach(), best_metric)
                    best_bounds = IntervalState(
                        torch.where(improve.unsqueeze(1), bounds.lower.detach(), best_bounds.lower),
                        torch.where(improve.unsqueeze(1), bounds.upper.detach(), best_bounds.upper),
                    )
                    for name, cur in alpha.items():
                        mask = improve.view(batch, *([1] * (cur.dim() - 1)))
                        best_alpha[name] = torch.where(mask, cur.detach(), best_alpha[name])
                    for name, cur in beta.items():
                        mask = improve.view(batch, *([1] * (cur.dim() - 1)))
                        best_beta[name] = torch.where(mask, cur.detach(), best_beta[name])
            if float(metric.detach().item()) > float(best_metric_scalar.item()):
                best_metric_scalar = metric.detach().clone()
                if not per_batch_params:
                    best_metric = metric_b.detach().clone()
                    best_bounds = IntervalState(bounds.lower.detach().clone(), bounds.upper.detach().clone())
                    best_alpha = {k: v.detach().clone() for k, v in alpha.items()}
                    best_beta = {k: v.detach().clone() for k, v in beta.items()}
        if step == int(steps):
            break
        loss = -metric_b.sum() if per_batch_params else -metric_b.mean()
        if not loss.requires_grad:
            break
        opt.zero_grad(set_to_none=True)
        loss.backward()
        if record is not None:
            def moments(p, key):
                st = opt.state.get(p, {})
                return st[key].detach().clone() if key in st else torch.zeros_like(p)
            rec = record[-1]
            rec["grad_alpha"] = {k: (v.grad.detach().clone() if v.grad is not None else None) for k, v in alpha.items()}
            rec["grad_beta"] = {k: (v.grad.detach().clone() if v.grad is not None else None) for k, v in beta.items()}
            rec["exp_avg"] = {("alpha", k): moments(v, "exp_avg") for k, v in alpha.items()}
            rec["exp_avg"].update({("beta", k): moments(v, "exp_avg") for k, v in beta.items()})
            rec["exp_avg_sq"] = {("alpha", k): moments(v, "exp_avg_sq") for k, v in alpha.items()}
            rec["exp_avg_sq"].update({("beta", k): moments(v, "exp_avg_sq") for k, v in beta.items()})
            rec["adam_step"] = step + 1
        opt.step()
        with torch.no_grad():
            for a in alpha.values():
                a.clamp_(0.0, 1.0)
            for b in beta.values():
                b.clamp_(0.0)
        if record is not None:
            record[-1]["alpha_next"] = {k: v.detach().clone() for k, v in alpha.items()}
            record[-1]["beta_next"] = {k: v.detach().clone() for k, v in beta.items()}
    out = (best_bounds, best_alpha, best_beta, choices)
    return out + ("unknown",) if return_feasibility else out


def run_alpha_crown(
    module: BFTaskModule,
    input_spec,
    *,
    linear_spec_C: Optional[torch.Tensor] = None,
    steps: int = 20,
    lr: float = 0.2,
    alpha_init: float = 0.5,
    relu_split_state=None,
    warm_start: Optional[Dict[str, torch.Tensor]] = None,
    objective: str = "lower",
    spec_reduce: str = "mean",
    soft_tau: float = 1.0,
    lb_weight: float = 1.0,
    ub_weight: float = 1.0,
):
    """alpha_crown.py:137-261 (shared alpha per ReLU); ``warm_start`` seeds alpha
    per ReLU input (alpha_crown.py:42-60).  The metric and loss of each objective
    reduce over the whole [B, S] bound (alpha_crown.py:62-135): "mean" is the
    mean of every element, "min"/"softmin" the batch mean of per-row reductions."""

    def reduce_specs(x, direction):
        if x.dim() != 2 or spec_reduce == "mean":
            return x.mean()
        if spec_reduce == "min":
            return (x.min(dim=1).values if direction == "min" else x.max(dim=1).values).mean()
        if spec_reduce == "softmin":
            tau = float(soft_tau)
            if tau <= 0.0:
                raise ValueError(f"soft_tau must be >0, got {soft_tau}")
            if direction == "min":
                return (-tau * torch.logsumexp(-x / tau, dim=1)).mean()
            return (tau * torch.logsumexp(x / tau, dim=1)).mean()
        raise AssertionError(f"unreachable spec_reduce: {spec_reduce}")

    def metric_of(bounds):
        if objective == "lower":
            return reduce_specs(bounds.lower, "min")
        if objective == "upper":
            return -reduce_specs(bounds.upper, "max")
        if objective == "gap":
            return -reduce_specs(bounds.upper - bounds.lower, "max")
        if objective == "both":
            return (float(lb_weight) * reduce_specs(bounds.lower, "min")
                    - float(ub_weight) * reduce_specs(bounds.upper, "max"))
        raise AssertionError(f"unreachable objective: {objective}")

    spec = normalize_input_spec(input_spec)
    interval_env, relu_pre = forward_ibp_trace(module, spec, relu_split_state=relu_split_state)
    alpha = {}
    for k, p in relu_pre.items():
        shape = tuple(int(d) for d in p.lower.shape[1:])
        if warm_start is not None and k in warm_start:
            a = warm_start[k].to(dtype=spec.center.dtype).reshape(shape).detach().clone()
        else:
            a = torch.full(shape, float(alpha_init), dtype=spec.center.dtype)
        alpha[k] = a.requires_grad_(True)
    opt = torch.optim.Adam(list(alpha.values()), lr=float(lr))
    best_metric = None
    best_bounds = None
    best_alpha = None
    for step in range(int(steps) + 1):
        bounds = crown_backward_from_trace(module, spec, interval_env=interval_env, relu_pre=relu_pre,
                                           linear_spec_C=linear_spec_C, relu_alpha=alpha)
        metric = metric_of(bounds)
        mv = float(metric.detach().item())
        if best_metric is None or mv > float(best_metric.item()):
            best_metric = metric.detach()
            best_bounds = IntervalState(bounds.lower.detach().clone(), bounds.upper.detach().clone())
            best_alpha = {k: v.detach().clone() for k, v in alpha.items()}
        if step == int(steps):
            break
        loss = -metric
        if not loss.requires_grad:   # no ambiguous ReLU left (alpha_crown.py:240-241)
            break
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
        with torch.no_grad():
            for a in alpha.values():
                a.clamp_(0.0, 1.0)
    return best_bounds, best_alpha


def domain_feasible(module: BFTaskModule, spec: InputSpec, relu_split_state: Dict[str, torch.Tensor]) -> torch.Tensor:
    """Per-domain IBP feasibility: True where the one-domain forward trace of
    crown_ibp.py:101-342 with that domain's split does not raise."""
    batch = int(spec.center.shape[0])
    ok = torch.zeros(batch, dtype=torch.bool)
    for d in range(batch):
        sub = InputSpec(value_name=spec.value_name, center=spec.center[d:d + 1], perturbation=spec.perturbation)
        try:
            forward_ibp_trace(module, sub, relu_split_state={k: v[d:d + 1] for k, v in relu_split_state.items()})
            ok[d] = True
        except ValueError:
            ok[d] = False
    return ok


def evaluate_domain_batch(
    module: BFTaskModule,
    spec: InputSpec,
    *,
    linear_spec_C: torch.Tensor,
    relu_split_state: Dict[str, torch.Tensor],
    steps: int,
    lr: float,
    alpha_init: float = 0.5,
    beta_init: float = 0.0,
    threshold: float = 0.0,
    tol: float = 1e-6,
    record: Optional[list] = None,
):
    """Node-batch evaluation of a BaB frontier (bab.py:1250-1460 + :870-895).

    Domains whose split empties an interval are rejected (closed), as the
    reference's per-node fallback does; the rest are evaluated in one
    ``per_batch_params=True`` alpha-beta call.  Returns a dict with per-domain
    ``feasible``, ``lower`` [D,S], ``upper``, ``certified`` and ``branch``.
    ``record`` receives the optimisation's per-step record over the feasible
    domains (``run_alpha_beta_crown``).
    """
    feasible = domain_feasible(module, spec, relu_split_state)
    idx = feasible.nonzero(as_tuple=False).flatten()
    D = int(spec.center.shape[0])
    S = int(linear_spec_C.shape[1])
    lower = torch.full((D, S), float("nan"), dtype=spec.center.dtype)
    upper = torch.full((D, S), float("nan"), dtype=spec.center.dtype)
    branch: List[Optional[Tuple[str, int]]] = [None] * D
    if idx.numel() > 0:
        sub_spec = InputSpec(value_name=spec.value_name, center=spec.center[idx], perturbation=spec.perturbation)
        sub_split = {k: v[idx] for k, v in relu_split_state.items()}
        bounds, _a, _b, choices = run_alpha_beta_crown(
            module, sub_spec, linear_spec_C=linear_spec_C[idx], relu_split_state=sub_split,
            steps=steps, lr=lr, alpha_init=alpha_init, beta_init=beta_init, per_batch_params=True, record=record,
        )
        lower[idx] = bounds.lower
        upper[idx] = bounds.upper
        for j, d in enumerate(idx.tolist()):
            branch[d] = choices[j]
    certified = torch.zeros(D, dtype=torch.bool)
    certified[idx] = lower[idx].min(dim=1).values >= float(threshold) - float(tol)
    return {"feasible": feasible, "lower": lower, "upper": upper, "certified": certified, "branch": branch}
