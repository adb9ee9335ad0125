"""CPU restatement of the reference's branch-and-bound loop (test infrastructure only).

Only tests, the smoke check and the bench's CPU baseline use this module, as
the checker; nothing in ``boundflow_amd`` imports it.

Follows ``solve_bab_mlp`` (boundflow/runtime/bab.py:631-1528) for the paths it
takes without a query recorder/runtime or node cache hits (a search tree never
evaluates the same split set twice, so the cache cannot hit):

* one search tree per example; heap keyed (priority, node_id), roots at -inf
  (:700-720); pop up to ``node_batch_size`` nodes per round for the alpha-beta
  oracle, one otherwise, skipping decided examples and charging the node
  budget (:957-977);
* a single popped node is evaluated alone (:995-1110), where the alpha-beta
  oracle first runs the first-layer split certificate (alpha_beta_crown.py:694-714)
  and the 1-D input restriction may narrow or close it (:1000-1012, :524-628);
  several together with per-node parameters and warm starts (:1250-1345), after
  the optional first-layer pre-pruning (:373-425); when the batched call raises
  (an IBP-infeasible split) every node is evaluated alone, certificate included,
  and the infeasible ones are rejected (:1399-1456);
* ``_process_evaluated_node`` (:870-955): best bounds, certification at
  min lb >= threshold - tol, branch on the evaluation's hint (alpha-beta) or
  the widest ambiguous IBP neuron (``_pick_branch``, :488-522), "unsafe" when
  none is left, "unknown" on the node budget, children left (-1) then right
  (+1) warm-started from the node's best alpha/beta;
* final statuses and aggregation (:365-371, :1488-1528).

Pinned by the reference-generated fixtures ``bab_solve_*`` (tests/golden) and,
in ``tests/test_oracle_bab.py``, by the soundness of a "proven" verdict on
sampled points and by the existence of a violating point for "unsafe".
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

from boundflow_amd.spec import BoxPerturbation, InputSpec, normalize_input_spec

from . import alpha_beta_ref as ab
from .crown_ref import forward_ibp_trace


@dataclass(order=True)
class _Item:
    priority: float
    node_id: int
    example_idx: int = field(compare=False)
    split: Dict[str, torch.Tensor] = field(compare=False)
    warm_alpha: Optional[Dict[str, torch.Tensor]] = field(compare=False, default=None)
    warm_beta: Optional[Dict[str, torch.Tensor]] = field(compare=False, default=None)


def _slice_spec(spec: InputSpec, idx: List[int]) -> InputSpec:
    p = spec.perturbation
    if isinstance(p, BoxPerturbation):
        return InputSpec.box(value_name=spec.value_name, lower=p.lower[idx], upper=p.upper[idx])
    return InputSpec(value_name=spec.value_name, center=spec.center[idx], perturbation=p)


class NodeInfeasible(ValueError):
    """A node whose splits the first-layer certificate proves infeasible: the
    reference closes it exactly as it closes one whose IBP trace raises
    (bab.py:1058-1069, :1421-1431)."""


def _objective_kw(cfg) -> dict:
    """The objective options BabConfig forwards to every oracle call (bab.py:147-151,
    :461-466, :1095-1100, :1334-1339)."""
    return {"objective": cfg.get("objective", "lower"), "spec_reduce": cfg.get("spec_reduce", "mean"),
            "soft_tau": float(cfg.get("soft_tau", 1.0)), "lb_weight": float(cfg.get("lb_weight", 1.0)),
            "ub_weight": float(cfg.get("ub_weight", 1.0))}


def _eval_single(module, spec, C, item: _Item, cfg):
    """eval_bab_alpha_beta_node / run_alpha_crown_mlp for one node; raises ValueError when
    the IBP trace is infeasible and NodeInfeasible when the certificate closes the node."""
    split = {k: v.unsqueeze(0) for k, v in item.split.items()}
    if cfg["oracle"] == "alpha_beta":
        bounds, alpha, beta, choices, feas = ab.run_alpha_beta_crown(
            module, spec, linear_spec_C=C, relu_split_state=split, steps=cfg["alpha_steps"], lr=cfg["alpha_lr"],
            alpha_init=cfg["alpha_init"], beta_init=cfg["beta_init"], warm_start_alpha=item.warm_alpha,
            warm_start_beta=item.warm_beta, return_feasibility=True, **_objective_kw(cfg))
        if feas == "infeasible":
            raise NodeInfeasible("first-layer split certificate")
        hint = choices[0] if len(choices) == 1 else None
        return bounds, alpha, beta, hint
    bounds, alpha = ab.run_alpha_crown(module, spec, linear_spec_C=C, steps=cfg["alpha_steps"], lr=cfg["alpha_lr"],
                                       alpha_init=cfg["alpha_init"], relu_split_state=split,
                                       warm_start=item.warm_alpha, **_objective_kw(cfg))
    return bounds, alpha, None, None


def restrict_1d_linf(module, spec: InputSpec, split: Dict[str, torch.Tensor]) -> Optional[InputSpec]:
    """bab.py:524-628: a one-input Linf spec narrowed by the first-layer split
    constraints s * (w_i x + b_i) >= 0 of linear layers reading the input; None
    when they leave nothing.  Any other spec is returned unchanged."""
    from boundflow_amd.spec import LpBallPerturbation
    if spec.center.dim() != 2 or int(spec.center.shape[1]) != 1:
        return spec
    p = spec.perturbation
    if not isinstance(p, LpBallPerturbation) or p.normalized_p() != "inf":
        return spec
    if int(spec.center.shape[0]) != 1:
        return spec
    task = module.get_entry_task()
    params = module.params
    x0 = float(spec.center[0, 0].item())
    eps = float(p.eps)
    lo, hi = x0 - eps, x0 + eps
    for op in task.ops:
        if op.op_type != "relu":
            continue
        x = op.inputs[0]
        sv = split.get(x)
        if sv is None:
            continue
        prod = next((q for q in task.ops if x in q.outputs), None)
        if prod is None or prod.op_type != "linear" or not prod.inputs or prod.inputs[0] != spec.value_name:
            continue
        W = params.get(prod.inputs[1])
        if W is None or W.dim() != 2 or int(W.shape[1]) != 1:
            continue
        if len(prod.inputs) == 3:
            b = params.get(prod.inputs[2])
            if b is None or b.dim() != 1 or int(b.shape[0]) != int(W.shape[0]):
                continue
        else:
            b = torch.zeros(int(W.shape[0]), dtype=W.dtype)
        for i in range(int(sv.shape[0])):
            sg = int(sv[i].item())
            if sg == 0:
                continue
            wi = float(W[i, 0].item())
            bi = float(b[i].item())
            if wi == 0.0:
                if (sg > 0 and bi < 0.0) or (sg < 0 and bi > 0.0):
                    return None
                continue
            t = -bi / wi
            if (sg > 0) == (wi > 0):
                lo = max(lo, t)
            else:
                hi = min(hi, t)
        if lo > hi:
            return None
    center = torch.tensor([[0.5 * (lo + hi)]], dtype=spec.center.dtype)
    return InputSpec.linf(value_name=spec.value_name, center=center, eps=float(0.5 * (hi - lo)))


def _pick_branch(module, spec, split: Dict[str, torch.Tensor]) -> Optional[Tuple[str, int]]:
    _env, pre = forward_ibp_trace(module, spec, relu_split_state={k: v.unsqueeze(0) for k, v in split.items()})
    return ab.branch_choices(pre)[0]


def solve_bab_mlp(module, input_spec, *, linear_spec_C, config) -> dict:
    cfg = dict(config)
    spec = normalize_input_spec(input_spec)
    # bab.py:656-659: the alpha oracle does not take conv graphs
    if any(op.op_type in ("conv2d", "flatten") for op in module.get_entry_task().ops) and cfg["oracle"] != "alpha_beta":
        raise NotImplementedError("alpha-only BaB does not yet support conv graphs")
    E = int(spec.center.shape[0])
    _env, pre0 = forward_ibp_trace(module, _slice_spec(spec, [0]))
    shapes = {k: tuple(int(d) for d in v.lower.shape[1:]) for k, v in pre0.items()}
    heap: List[_Item] = []
    live = [0] * E
    visited = [0] * E
    evaluated = [0] * E
    expanded = [0] * E
    best_lower = [float("-inf")] * E
    best_upper = [float("inf")] * E
    status: List[Optional[str]] = [None] * E
    node_id = 0
    for e in range(E):
        split = {k: torch.zeros(s, dtype=torch.int8) for k, s in shapes.items()}
        heapq.heappush(heap, _Item(float("-inf"), node_id, e, split))
        node_id += 1
        live[e] = 1
    batch_rounds = 0
    popped_total = 0
    max_q = len(heap)
    do_batch = (cfg["oracle"] == "alpha_beta" and int(cfg["node_batch_size"]) > 1
                and not cfg.get("use_1d_linf_input_restriction_patch", False))
    prune = bool(cfg.get("enable_batch_infeasible_prune", False)) and cfg["oracle"] == "alpha_beta"

    def done_if_empty(e):
        if status[e] is None and live[e] == 0:
            status[e] = "proven"

    def process(item: _Item, bounds, alpha, beta, hint):
        nonlocal node_id, max_q
        e = item.example_idx
        evaluated[e] += 1
        node_lower = float(bounds.lower.min().item())
        node_upper = float(bounds.upper.max().item())
        best_lower[e] = max(best_lower[e], node_lower)
        best_upper[e] = min(best_upper[e], node_upper)
        live[e] = max(0, live[e] - 1)
        if status[e] is not None:
            return
        if node_lower >= float(cfg["threshold"]) - float(cfg["tol"]):
            done_if_empty(e)
            return
        branch = hint if (cfg["oracle"] == "alpha_beta" and cfg["use_branch_hint"]) else None
        if branch is None:
            branch = _pick_branch(module, _slice_spec(spec, [e]), item.split)
        if branch is None:
            status[e] = "unsafe"
            return
        if visited[e] >= int(cfg["max_nodes"]):
            status[e] = "unknown"
            return
        name, idx = branch
        for val in (-1, 1):
            child = {k: v.clone() for k, v in item.split.items()}
            child[name].reshape(-1)[int(idx)] = val
            wa = {k: v.detach().clone() for k, v in alpha.items()}
            wb = None if beta is None else {k: v.detach().clone() for k, v in beta.items()}
            heapq.heappush(heap, _Item(node_lower, node_id, e, child, wa, wb))
            node_id += 1
        live[e] += 2
        expanded[e] += 1
        max_q = max(max_q, len(heap))

    while heap and any(s is None for s in status):
        want = int(cfg["node_batch_size"]) if do_batch else 1
        items: List[_Item] = []
        while len(items) < want and heap:
            item = heapq.heappop(heap)
            e = item.example_idx
            if status[e] is not None:
                continue
            if visited[e] >= int(cfg["max_nodes"]):
                status[e] = "unknown"
                live[e] = 0
                continue
            visited[e] += 1
            items.append(item)
        if not items:
            break
        if do_batch:
            batch_rounds += 1
            popped_total += len(items)
        results: Dict[int, tuple] = {}
        if len(items) == 1:
            item = items[0]
            e = item.example_idx
            C = None if linear_spec_C is None else linear_spec_C[[e]]
            node_spec = _slice_spec(spec, [e])
            if cfg.get("use_1d_linf_input_restriction_patch", False):
                node_spec = restrict_1d_linf(module, node_spec, item.split)
                if node_spec is None:
                    live[e] = max(0, live[e] - 1)
                    done_if_empty(e)
                    continue
            try:
                results[0] = _eval_single(module, node_spec, C, item, cfg)
            except ValueError:
                live[e] = max(0, live[e] - 1)
                done_if_empty(e)
                continue
        else:
            # per-node first-layer pre-pruning (bab.py:373-425, applied at :1157-1168)
            keep = []
            for j, item in enumerate(items):
                e = item.example_idx
                if prune and ab.split_certificate(module, _slice_spec(spec, [e]),
                                                  {k: v.unsqueeze(0) for k, v in item.split.items()})[0]:
                    live[e] = max(0, live[e] - 1)
                    done_if_empty(e)
                else:
                    keep.append(j)
            sub_items = [items[j] for j in keep]
            results.update(_eval_batch(module, spec, linear_spec_C, sub_items, keep, shapes, cfg, live,
                                       done_if_empty))
        for j, item in enumerate(items):
            if j in results:
                process(item, *results[j])

    for e in range(E):
        if status[e] is None:
            status[e] = "proven" if live[e] == 0 else "unknown"
    agg = "unsafe" if any(s == "unsafe" for s in status) else ("proven" if all(s == "proven" for s in status)
                                                               else "unknown")
    nbs = int(cfg["node_batch_size"])
    return {
        "status": agg, "nodes_visited": sum(visited), "nodes_evaluated": sum(evaluated),
        "nodes_expanded": sum(expanded), "max_queue": max_q, "batch_rounds": batch_rounds,
        "avg_batch_fill_rate": 0.0 if nbs <= 1 or batch_rounds == 0 else popped_total / float(batch_rounds * nbs),
        "per_status": status, "per_visited": visited, "per_evaluated": evaluated, "per_expanded": expanded,
        "per_best_lower": best_lower, "per_best_upper": best_upper,
    }


def _eval_batch(module, spec, linear_spec_C, items, slots, shapes, cfg, live, done_if_empty) -> Dict[int, tuple]:
    """bab.py:1250-1456: one per_batch_params call over the nodes; when it raises (an
    IBP-infeasible split) every node is evaluated alone (with the single-node
    certificate) and the infeasible ones are closed.  Results keyed by ``slots``."""
    results: Dict[int, tuple] = {}
    if not items:
        return results
    ex = [it.example_idx for it in items]
    split_b = {k: torch.stack([it.split[k] for it in items]) for k in shapes}
    warm_a = {k: torch.stack([it.warm_alpha[k].reshape(shapes[k]) if it.warm_alpha is not None
                              else torch.full(shapes[k], float(cfg["alpha_init"]), dtype=spec.center.dtype)
                              for it in items]) for k in shapes}
    warm_b = {k: torch.stack([it.warm_beta[k].reshape(shapes[k]) if it.warm_beta is not None
                              else torch.full(shapes[k], float(cfg["beta_init"]), dtype=spec.center.dtype)
                              for it in items]) for k in shapes}
    C = None if linear_spec_C is None else linear_spec_C[ex]
    try:
        bounds, alpha, beta, choices = ab.run_alpha_beta_crown(
            module, _slice_spec(spec, ex), linear_spec_C=C, relu_split_state=split_b,
            steps=cfg["alpha_steps"], lr=cfg["alpha_lr"], alpha_init=cfg["alpha_init"],
            beta_init=cfg["beta_init"], warm_start_alpha=warm_a, warm_start_beta=warm_b,
            per_batch_params=True, **_objective_kw(cfg))
        if len(items) == 1 and choices is None:
            # one node left after pruning: the batched call's own certificate closed it
            live[ex[0]] = max(0, live[ex[0]] - 1)
            done_if_empty(ex[0])
            return results
        for j in range(len(items)):
            nb = type(bounds)(bounds.lower[j:j + 1].clone(), bounds.upper[j:j + 1].clone())
            results[slots[j]] = (nb, {k: v[j].clone() for k, v in alpha.items()},
                                 {k: v[j].clone() for k, v in beta.items()}, choices[j])
    except ValueError:
        for j, item in enumerate(items):
            e = item.example_idx
            C1 = None if linear_spec_C is None else linear_spec_C[[e]]
            try:
                results[slots[j]] = _eval_single(module, _slice_spec(spec, [e]), C1, item, cfg)
            except ValueError:
                live[e] = max(0, live[e] - 1)
                done_if_empty(e)
    return results


# ---------------------------------------------------------------------------
# The native ReLU-split queue (boundflow/runtime/native_relu_split_bab_runtime.py:592-789)


def native_priority(lower: float) -> float:
    """native_relu_split_bab_runtime.py:1128-1131: the lower bound to 7 significant digits."""
    if not torch.isfinite(torch.tensor(lower)):
        raise ValueError("native ReLU-split queue bound must be finite")
    return float(f"{lower:.7g}")


def native_select_branch(relu_pre, split: Dict[str, torch.Tensor]):
    """native_relu_split_bab_runtime.py:1015-1049: the widest unsplit ambiguous neuron
    (width upper - lower in Python floats), ties to the first ReLU name in sorted
    order, then the lowest index; (name, index, lower, upper, width) or None."""
    best = None
    for name in sorted(relu_pre):
        lo = relu_pre[name].lower.reshape(-1).tolist()
        hi = relu_pre[name].upper.reshape(-1).tolist()
        sp = split[name].reshape(-1).tolist()
        for i, (l, u, s) in enumerate(zip(lo, hi, sp)):
            if int(s) == 0 and l < 0.0 < u:
                key = (-(u - l), name, i)
                if best is None or key < best[0]:
                    best = (key, (name, i, l, u, u - l))
    return None if best is None else best[1]


def native_adaptive_alpha(relu_pre) -> Dict[str, torch.Tensor]:
    """The ADAPTIVE lower slope of the native plain-CROWN relaxation
    (boundflow/runtime/bound_ir_interpreter.py:1380-1397): on an ambiguous neuron
    alpha_l = 1(u / max(u - l, eps) > 0.5), the upper chord's slope above one half."""
    out = {}
    for name, pre in relu_pre.items():
        lo, hi = pre.lower, pre.upper
        amb = (lo < 0) & (hi > 0)
        a = torch.zeros_like(lo)
        a[lo >= 0] = 1.0
        den = (hi[amb] - lo[amb]).clamp_min(torch.finfo(lo.dtype).eps)
        a[amb] = (hi[amb] / den > 0.5).to(lo.dtype)
        out[name] = a
    return out


def run_native_relu_split_bab(module, input_spec, *, linear_spec_C, run_id: str, max_nodes: int, max_depth: int,
                              expansion_batch_size: int, max_eval_batch_size: int, threshold: float = 0.0) -> dict:
    """The bounded best-first queue of native_relu_split_bab_runtime.py:592-789.

    Nodes are evaluated in batches of at most ``max_eval_batch_size``: CROWN with the
    ADAPTIVE lower slope (``native_adaptive_alpha``) on the box input repeated per
    node, the node's splits applied to its IBP pre-activation boxes; the root
    first, then every round's children together.
    A round pops up to ``expansion_batch_size`` entries (priority, serial, node id)
    and for each: prune when lower >= threshold, terminal at the depth limit or
    without a branch, stop when two more nodes would exceed ``max_nodes`` (the
    rest of the round goes back to the heap), else expand into the inactive (-1)
    then active (+1) child.  Children are pushed with the serial the round ends
    with.  Returns the evaluations, decisions, final frontier, status and the
    largest queue."""
    spec = normalize_input_spec(input_spec)
    if not isinstance(spec.perturbation, BoxPerturbation):
        raise NotImplementedError("native ReLU-split BaB v1 requires a box input")
    lo0, hi0 = spec.perturbation.lower, spec.perturbation.upper
    C = linear_spec_C if linear_spec_C.dim() == 2 else linear_spec_C[0]
    _env, root_pre = forward_ibp_trace(module, spec)
    names = sorted(root_pre)
    shapes = {n: tuple(int(d) for d in root_pre[n].lower.shape[1:]) for n in names}
    nodes: Dict[str, dict] = {}
    evaluations: List[dict] = []
    decisions: List[dict] = []
    serial = {"next": 1, "stacks": 0}

    def evaluate(batch: List[dict]) -> None:
        for start in range(0, len(batch), max_eval_batch_size):
            chunk = batch[start:start + max_eval_batch_size]
            k = len(chunk)
            bspec = InputSpec.box(value_name=spec.value_name, lower=lo0.repeat((k,) + (1,) * (lo0.dim() - 1)),
                                  upper=hi0.repeat((k,) + (1,) * (hi0.dim() - 1)))
            split_b = {n: torch.stack([c["split"][n] for c in chunk]) for n in names}
            _e, pre = forward_ibp_trace(module, bspec, relu_split_state=split_b)
            from .crown_ref import crown_backward_from_trace
            b = crown_backward_from_trace(module, bspec, interval_env=_e, relu_pre=pre,
                                          linear_spec_C=C.unsqueeze(0).expand(k, -1, -1),
                                          relu_alpha=native_adaptive_alpha(pre))
            serial["stacks"] += 1
            for j, c in enumerate(chunk):
                node_pre = {n: type(pre[n])(pre[n].lower[j:j + 1], pre[n].upper[j:j + 1]) for n in names}
                c["branch"] = native_select_branch(node_pre, c["split"])
                c["lower"] = float(b.lower[j, 0].item())
                c["upper"] = float(b.upper[j, 0].item())
                c["priority"] = native_priority(c["lower"])
                evaluations.append({k2: c[k2] for k2 in ("node_id", "parent", "depth", "lower", "upper",
                                                          "priority", "branch")})

    root = {"node_id": f"{run_id}:n000000", "parent": None, "depth": 0,
            "split": {n: torch.zeros(shapes[n], dtype=torch.int8) for n in names}}
    nodes[root["node_id"]] = root
    evaluate([root])
    heap = [(root["priority"], 0, root["node_id"])]
    max_q = 1
    exhausted = False
    while heap and not exhausted:
        selected = [heapq.heappop(heap) for _ in range(min(expansion_batch_size, len(heap)))]
        generated: List[dict] = []
        for pos, entry in enumerate(selected):
            node = nodes[entry[2]]
            if node["lower"] >= threshold:
                decisions.append({"node_id": node["node_id"], "kind": "prune", "reason": "lower_bound_meets_threshold"})
                continue
            if node["depth"] >= max_depth:
                decisions.append({"node_id": node["node_id"], "kind": "terminal", "reason": "configured_depth_limit"})
                continue
            br = node["branch"]
            if br is None:
                decisions.append({"node_id": node["node_id"], "kind": "terminal", "reason": "no_unsplit_ambiguous_relu"})
                continue
            if len(evaluations) + len(generated) + 2 > max_nodes:
                for pending in selected[pos:]:
                    heapq.heappush(heap, pending)
                exhausted = True
                break
            kids = []
            for val in (-1, 1):
                split = {n: v.clone() for n, v in node["split"].items()}
                split[br[0]].reshape(-1)[br[1]] = val
                kid = {"node_id": f"{run_id}:n{serial['next']:06d}", "parent": node["node_id"],
                       "depth": node["depth"] + 1, "split": split}
                serial["next"] += 1
                nodes[kid["node_id"]] = kid
                kids.append(kid)
            generated.extend(kids)
            decisions.append({"node_id": node["node_id"], "kind": "expand", "reason": "widest_unsplit_ambiguous_relu",
                              "children": [k["node_id"] for k in kids], "branch": br})
        if generated:
            evaluate(generated)
            for kid in generated:
                heapq.heappush(heap, (kid["priority"], serial["next"], kid["node_id"]))
            max_q = max(max_q, len(heap))
    frontier = [e[2] for e in sorted(heap, key=lambda e: (e[0], e[1]))]
    return {"status": "budget_exhausted" if exhausted else "complete", "evaluations": evaluations,
            "decisions": decisions, "frontier": frontier, "max_queue_size": max_q, "stacks": serial["stacks"]}
