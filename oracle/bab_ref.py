"""CPU restatement of the reference's branch-and-bound loop (test infrastructure only).

Only tests, the smoke check and the bench's CPU baseline use this module, as
the checker; nothing in ``boundflow_amd`` imports it.

Follows ``solve_bab_mlp`` (boundflow/runtime/bab.py:631-1528) for the paths it
takes without a query recorder/runtime, node cache hits, the 1-D input
restriction or first-layer pre-pruning:

* one search tree per example; heap keyed (priority, node_id), roots at -inf
  (:700-720); pop up to ``node_batch_size`` nodes per round for the alpha-beta
  oracle, one otherwise, skipping decided examples and charging the node
  budget (:957-977);
* a single popped node is evaluated alone (:995-1110), several together with
  per-node parameters and warm starts (:1250-1345); when the batched call
  raises (an infeasible split) every node is evaluated alone and the
  infeasible ones are rejected (:1399-1456);
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


def _eval_single(module, spec, C, item: _Item, cfg):
    """eval_bab_alpha_beta_node / run_alpha_crown_mlp for one node; raises ValueError when infeasible."""
    split = {k: v.unsqueeze(0) for k, v in item.split.items()}
    if cfg["oracle"] == "alpha_beta":
        bounds, alpha, beta, choices = ab.run_alpha_beta_crown(
            module, spec, linear_spec_C=C, relu_split_state=split, steps=cfg["alpha_steps"], lr=cfg["alpha_lr"],
            alpha_init=cfg["alpha_init"], beta_init=cfg["beta_init"], warm_start_alpha=item.warm_alpha,
            warm_start_beta=item.warm_beta)
        hint = choices[0] if len(choices) == 1 else None
        return bounds, alpha, beta, hint
    bounds, alpha = ab.run_alpha_crown(module, spec, linear_spec_C=C, steps=cfg["alpha_steps"], lr=cfg["alpha_lr"],
                                       alpha_init=cfg["alpha_init"], relu_split_state=split,
                                       warm_start=item.warm_alpha)
    return bounds, alpha, None, None


def _pick_branch(module, spec, split: Dict[str, torch.Tensor]) -> Optional[Tuple[str, int]]:
    _env, pre = forward_ibp_trace(module, spec, relu_split_state={k: v.unsqueeze(0) for k, v in split.items()})
    return ab.branch_choices(pre)[0]


def solve_bab_mlp(module, input_spec, *, linear_spec_C, config) -> dict:
    cfg = dict(config)
    spec = normalize_input_spec(input_spec)
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
    do_batch = cfg["oracle"] == "alpha_beta" and int(cfg["node_batch_size"]) > 1

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
            try:
                results[0] = _eval_single(module, _slice_spec(spec, [e]), C, item, cfg)
            except ValueError:
                live[e] = max(0, live[e] - 1)
                done_if_empty(e)
                continue
        else:
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
                    per_batch_params=True)
                for j in range(len(items)):
                    nb = type(bounds)(bounds.lower[j:j + 1].clone(), bounds.upper[j:j + 1].clone())
                    results[j] = (nb, {k: v[j].clone() for k, v in alpha.items()},
                                  {k: v[j].clone() for k, v in beta.items()}, choices[j])
            except ValueError:
                for j, item in enumerate(items):
                    e = item.example_idx
                    C1 = None if linear_spec_C is None else linear_spec_C[[e]]
                    try:
                        results[j] = _eval_single(module, _slice_spec(spec, [e]), C1, item, cfg)
                    except ValueError:
                        live[e] = max(0, live[e] - 1)
                        done_if_empty(e)
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
