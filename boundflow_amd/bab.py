"""HIP node-batch evaluation of a ReLU-split BaB frontier (beta-CROWN).

Counterpart of the batched section of ``solve_bab_mlp``
(boundflow/runtime/bab.py:1250-1460) and of ``execute_alpha_beta_query_batch``
(boundflow/runtime/query_executor.py:96-200): every domain of the batch carries
its own split vector, alpha and beta; one ``run_alpha_beta_crown_mlp`` call with
``per_batch_params=True`` optimises them all, and each domain is then closed
(certified: min_s lb >= threshold - tol, boundflow/runtime/bab.py:870-895),
closed as infeasible (its split empties a pre-activation box -- the reference
raises for the whole batch and re-evaluates node by node, rejecting such nodes,
bab.py:1400-1460), or left open with the branching decision of
alpha_beta_crown.py:145-182.  Domains are independent, so one infeasible domain
does not disturb the others.
"""

from __future__ import annotations

import heapq
import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from . import _lib
from .alpha_beta import branch_tensors, run_alpha_beta_crown_mlp, run_alpha_crown_mlp
from .crown import NotAChain, forward_ibp_trace, parse_chain
from .spec import BoxPerturbation, InputSpec, LpBallPerturbation, normalize_input_spec


def evaluate_domain_batch(module, input_spec, *, linear_spec_C: torch.Tensor,
                          relu_split_state: Dict[str, torch.Tensor], steps: int = 10, lr: float = 0.2,
                          alpha_init: float = 0.5, beta_init: float = 0.0,
                          warm_start_alpha: Optional[Dict[str, torch.Tensor]] = None,
                          warm_start_beta: Optional[Dict[str, torch.Tensor]] = None,
                          threshold: float = 0.0, tol: float = 1e-6, record: Optional[list] = None):
    """Returns a dict of device tensors: ``status`` int32 [D] (0 open, 1 certified,
    2 infeasible), ``lower``/``upper`` [D, S], ``branch_layer``/``branch_neuron``
    int32 [D] (-1 when no ambiguous neuron is left), ``alpha``/``beta`` per ReLU.
    ``record`` is passed to the optimiser (per-step parity diagnostics)."""
    spec = normalize_input_spec(input_spec)
    chain, _shapes, _has_conv = _relu_layout(module, spec)
    trace = forward_ibp_trace(module, spec, relu_split_state=relu_split_state, chain=chain,
                              raise_on_infeasible=False, relu_inputs_only=True)
    D = int(spec.center.shape[0])
    layer, neuron, _gap = branch_tensors(trace, D)
    bounds, alpha, beta, _stats = run_alpha_beta_crown_mlp(
        module, spec, linear_spec_C=linear_spec_C, relu_split_state=relu_split_state, steps=steps, lr=lr,
        alpha_init=alpha_init, beta_init=beta_init, warm_start_alpha=warm_start_alpha,
        warm_start_beta=warm_start_beta, per_batch_params=True, trace=trace, first_layer_certificate=False,
        record=record)
    S = int(bounds.lower.shape[1])
    status = torch.empty(D, dtype=torch.int32, device=spec.center.device)
    _lib.call("bf_domain_status", _lib.ptr(bounds.lower), D, S, _lib.ptr(trace.infeasible), float(threshold),
              float(tol), _lib.ptr(status), _lib.stream_handle())
    return {"status": status, "lower": bounds.lower, "upper": bounds.upper, "branch_layer": layer,
            "branch_neuron": neuron, "alpha": alpha, "beta": beta, "infeasible": trace.infeasible,
            "relu_names": list(trace.relu_pre.keys())}


def _relu_layout(module, spec):
    """(chain or None, per-sample shape of every ReLU input in op order, whether a conv2d
    is present) for a chain or a DAG task."""
    try:
        chain = parse_chain(module, spec)
    except NotAChain:
        from .crown_dag import relu_input_shapes
        task = module.get_entry_task()
        return None, relu_input_shapes(module, spec), any(op.op_type == "conv2d" for op in task.ops)
    return chain, dict(chain.relu_shapes), any(layer.kind == "conv2d" for layer in chain.layers)


# ---------------------------------------------------------------------------
# Branch and bound over a device-resident frontier


@dataclass(frozen=True)
class BabConfig:
    """Search options, field for field as the reference's BabConfig (bab.py:134-153)."""

    max_nodes: int = 10_000
    oracle: str = "alpha"
    use_1d_linf_input_restriction_patch: bool = False
    node_batch_size: int = 1
    use_branch_hint: bool = True
    enable_node_eval_cache: bool = True
    enable_batch_infeasible_prune: bool = False
    alpha_steps: int = 20
    alpha_lr: float = 0.2
    alpha_init: float = 0.5
    beta_init: float = 0.0
    objective: str = "lower"
    spec_reduce: str = "mean"
    soft_tau: float = 1.0
    lb_weight: float = 1.0
    ub_weight: float = 1.0
    threshold: float = 0.0
    tol: float = 1e-6


@dataclass(frozen=True)
class BabPerExampleResult:
    example_idx: int
    status: str
    nodes_visited: int
    nodes_evaluated: int
    nodes_expanded: int
    best_lower: float
    best_upper: float


@dataclass(frozen=True)
class BabResult:
    status: str
    nodes_visited: int
    nodes_evaluated: int
    nodes_expanded: int
    max_queue: int
    batch_rounds: int
    avg_batch_fill_rate: float
    best_lower: float
    best_upper: float
    per_example: Tuple[BabPerExampleResult, ...] = ()


def _aggregate_status(statuses: List[str]) -> str:
    if any(s == "unsafe" for s in statuses):
        return "unsafe"
    if all(s == "proven" for s in statuses):
        return "proven"
    return "unknown"


class _Frontier:
    """Split vectors and warm-start alpha/beta of the open nodes, one device row
    per node slot (int8 splits, fp32 parameters), grown by doubling; freed slots
    are reused."""

    def __init__(self, sizes: Dict[str, int], dev, capacity: int = 64):
        self.sizes = sizes
        self.dev = dev
        self.cap = capacity
        self.split = {n: torch.zeros(capacity, k, dtype=torch.int8, device=dev) for n, k in sizes.items()}
        self.alpha = {n: torch.zeros(capacity, k, device=dev) for n, k in sizes.items()}
        self.beta = {n: torch.zeros(capacity, k, device=dev) for n, k in sizes.items()}
        self.free: List[int] = list(range(capacity - 1, -1, -1))

    def alloc(self, count: int) -> List[int]:
        while len(self.free) < count:
            old = self.cap
            self.cap *= 2
            for d in (self.split, self.alpha, self.beta):
                for n, t in d.items():
                    grown = torch.zeros((self.cap,) + tuple(t.shape[1:]), dtype=t.dtype, device=self.dev)
                    grown[:old] = t
                    d[n] = grown
            self.free.extend(range(self.cap - 1, old - 1, -1))
        return [self.free.pop() for _ in range(count)]

    def release(self, slots: List[int]) -> None:
        self.free.extend(slots)


def solve_bab_mlp(module, input_spec, *, linear_spec_C: Optional[torch.Tensor] = None,
                  config: Optional[BabConfig] = None) -> BabResult:
    """HIP counterpart of solve_bab_mlp (boundflow/runtime/bab.py:631-1528).

    One search tree per input example; nodes are popped in the reference's
    heap order (parent lower bound, then creation order), up to
    ``node_batch_size`` per round for the alpha-beta oracle, and evaluated
    together.  Split vectors and warm-start parameters of every open node stay
    on the device; a round gathers them, runs one ``run_alpha_beta_crown_mlp``
    (per-node parameters) or, for the alpha oracle, one ``run_alpha_crown_mlp``,
    reads back the node lower/upper bounds, infeasibility and branching
    decisions in a single transfer, and writes the children's split vectors and
    warm starts (the parent's best alpha/beta) into free rows.  A node is
    closed when min_s lb >= threshold - tol, dropped when its splits are
    infeasible, and split on the widest ambiguous neuron otherwise; an example
    is "unsafe" when an open node has no ambiguous neuron left, "unknown" when
    its node budget runs out, "proven" when its tree empties.

    Nodes are closed as infeasible where the reference closes them: an IBP
    trace that empties a pre-activation box, and the first-layer split
    certificate (``split_certificate``) wherever the reference evaluates a node
    alone -- a round of one node, and every node of a batch that holds an
    IBP-infeasible node (the reference's per-node fallback, bab.py:1399-1456);
    with ``enable_batch_infeasible_prune`` the certificate also removes nodes
    from a batch before its evaluation (bab.py:373-425).  With
    ``use_1d_linf_input_restriction_patch`` a one-input Linf example's node is
    evaluated on its interval narrowed by the first-layer splits, and closed
    when they leave nothing (bab.py:524-628).

    A search tree never evaluates the same split set twice, so the reference's
    node-evaluation cache cannot hit and has no counterpart.  The objective
    options (objective, spec_reduce, soft_tau, lb_weight, ub_weight) go to every
    node evaluation, as the reference forwards them (bab.py:461-466, :1095-1100,
    :1334-1339); the node's verdict reads its lower bound whatever the objective.
    """
    cfg = config or BabConfig()
    if int(cfg.max_nodes) < 1:
        raise ValueError(f"max_nodes must be >=1, got {cfg.max_nodes}")
    if int(cfg.node_batch_size) < 1:
        raise ValueError(f"node_batch_size must be >=1, got {cfg.node_batch_size}")
    if cfg.oracle not in ("alpha", "alpha_beta"):
        raise ValueError(f"unknown BaB oracle: {cfg.oracle}")
    spec = normalize_input_spec(input_spec)
    module.validate()
    chain, relu_shapes, has_conv = _relu_layout(module, spec)
    if has_conv and cfg.oracle != "alpha_beta":
        raise NotImplementedError("alpha-only BaB does not yet support conv graphs")
    dev = spec.center.device
    E = int(spec.center.shape[0])
    sizes = {name: int(torch.tensor(shape).prod()) for name, shape in relu_shapes.items()}
    names = list(sizes)
    front = _Frontier(sizes, dev)
    threshold, tol = float(cfg.threshold), float(cfg.tol)

    heap: List[Tuple[float, int, int, int]] = []   # (priority, node_id, example, slot)
    live = [0] * E
    visited = [0] * E
    evaluated = [0] * E
    expanded = [0] * E
    best_lower = [float("-inf")] * E
    best_upper = [float("inf")] * E
    status: List[Optional[str]] = [None] * E
    node_id = 0
    roots = front.alloc(E)
    for e in range(E):
        slot = roots[e]
        for n in names:
            front.split[n][slot].zero_()
            front.alpha[n][slot].fill_(float(cfg.alpha_init))
            front.beta[n][slot].fill_(float(cfg.beta_init))
        heapq.heappush(heap, (float("-inf"), node_id, e, slot))
        node_id += 1
        live[e] = 1
    batch_rounds = 0
    popped_total = 0
    max_q = len(heap)
    do_batch = (cfg.oracle == "alpha_beta" and int(cfg.node_batch_size) > 1
                and not cfg.use_1d_linf_input_restriction_patch)

    def finish_if_empty(e: int) -> None:
        if status[e] is None and live[e] == 0:
            status[e] = "proven"

    while heap and any(s is None for s in status):
        want = int(cfg.node_batch_size) if do_batch else 1
        items: List[Tuple[float, int, int, int]] = []
        while len(items) < want and heap:
            item = heapq.heappop(heap)
            e = item[2]
            if status[e] is not None:
                front.release([item[3]])
                continue
            if visited[e] >= int(cfg.max_nodes):
                status[e] = "unknown"
                live[e] = 0
                front.release([item[3]])
                continue
            visited[e] += 1
            items.append(item)
        if not items:
            break
        if do_batch:
            batch_rounds += 1
            popped_total += len(items)
        out = _evaluate_nodes(module, spec, chain, relu_shapes, linear_spec_C, items, front, names, cfg)
        expansions: List[Tuple[int, int, int]] = []   # (row in this round, layer, neuron)
        child_meta: List[Tuple[int, float]] = []      # (example, priority) per expansion
        for row, item in enumerate(items):
            e = item[2]
            if out["closed"][row]:
                live[e] = max(0, live[e] - 1)
                finish_if_empty(e)
                continue
            evaluated[e] += 1
            node_lower = out["node_lower"][row]
            node_upper = out["node_upper"][row]
            best_lower[e] = max(best_lower[e], node_lower)
            best_upper[e] = min(best_upper[e], node_upper)
            live[e] = max(0, live[e] - 1)
            if status[e] is not None:
                continue
            if node_lower >= threshold - tol:
                finish_if_empty(e)
                continue
            layer = out["branch_layer"][row]
            if layer < 0:
                status[e] = "unsafe"
                continue
            if visited[e] >= int(cfg.max_nodes):
                status[e] = "unknown"
                continue
            expansions.append((row, layer, out["branch_neuron"][row]))
            child_meta.append((e, node_lower))
            live[e] += 2
            expanded[e] += 1
        if expansions:
            slots = front.alloc(2 * len(expansions))
            rows = torch.tensor([r for r, _l, _n in expansions for _ in (0, 1)], device=dev, dtype=torch.long)
            dst = torch.tensor(slots, device=dev, dtype=torch.long)
            for li, n in enumerate(names):
                front.split[n][dst] = out["split"][n][rows]
                front.alpha[n][dst] = out["alpha"][n][rows].to(torch.float32)
                front.beta[n][dst] = out["beta"][n][rows].to(torch.float32)
                sel = [(2 * i + side, nn, val) for i, (_r, lay, nn) in enumerate(expansions) if lay == li
                       for side, val in ((0, -1), (1, 1))]
                if sel:
                    si = torch.tensor([slots[k] for k, _nn, _v in sel], device=dev, dtype=torch.long)
                    ni = torch.tensor([nn for _k, nn, _v in sel], device=dev, dtype=torch.long)
                    vv = torch.tensor([v for _k, _nn, v in sel], device=dev, dtype=torch.int8)
                    front.split[n][si, ni] = vv
            for i, (e, prio) in enumerate(child_meta):
                heapq.heappush(heap, (prio, node_id, e, slots[2 * i]))       # left: inactive (-1)
                node_id += 1
                heapq.heappush(heap, (prio, node_id, e, slots[2 * i + 1]))   # right: active (+1)
                node_id += 1
            max_q = max(max_q, len(heap))
        front.release([item[3] for item in items])

    for e in range(E):
        if status[e] is None:
            status[e] = "proven" if live[e] == 0 else "unknown"
    per = tuple(BabPerExampleResult(example_idx=e, status=status[e] or "unknown", nodes_visited=visited[e],
                                    nodes_evaluated=evaluated[e], nodes_expanded=expanded[e],
                                    best_lower=best_lower[e], best_upper=best_upper[e]) for e in range(E))
    fill = 0.0 if int(cfg.node_batch_size) <= 1 or batch_rounds == 0 else \
        float(popped_total) / float(batch_rounds * int(cfg.node_batch_size))
    return BabResult(status=_aggregate_status([r.status for r in per]), nodes_visited=sum(visited),
                     nodes_evaluated=sum(evaluated), nodes_expanded=sum(expanded), max_queue=max_q,
                     batch_rounds=batch_rounds, avg_batch_fill_rate=fill,
                     best_lower=min(r.best_lower for r in per), best_upper=max(r.best_upper for r in per),
                     per_example=per)


def _objective_kw(cfg: BabConfig) -> dict:
    return {"objective": cfg.objective, "spec_reduce": cfg.spec_reduce, "soft_tau": float(cfg.soft_tau),
            "lb_weight": float(cfg.lb_weight), "ub_weight": float(cfg.ub_weight)}


def _evaluate_nodes(module, spec, chain, shapes, linear_spec_C, items, front: _Frontier, names, cfg: BabConfig):
    """One round: gather the popped nodes' inputs, splits and warm starts from
    the frontier, run the oracle on all of them, and return per node whether it
    is closed as infeasible, its lower/upper bound and branch decision on the
    host (one transfer; a second only in a round with an IBP-infeasible node of
    a batch), plus the gathered splits and the best alpha/beta on the device.

    Closing follows the reference: a node evaluated alone (a round of one node,
    or every node of a batch that holds an IBP-infeasible one) is closed by the
    first-layer certificate or its IBP trace; a node of an evaluated batch only
    by pre-pruning.  Every node is evaluated in the batch regardless: nodes do
    not interact, so a closed node's evaluation changes nothing for the others."""
    from .split_certificate import check_flags, split_certificate
    dev = spec.center.device
    ex = torch.tensor([it[2] for it in items], device=dev, dtype=torch.long)
    sl = torch.tensor([it[3] for it in items], device=dev, dtype=torch.long)
    b = len(items)
    pert = spec.perturbation
    if isinstance(pert, BoxPerturbation):
        sub = InputSpec.box(value_name=spec.value_name, lower=pert.lower[ex], upper=pert.upper[ex])
    else:
        sub = InputSpec(value_name=spec.value_name, center=spec.center[ex], perturbation=pert)
    split = {n: front.split[n][sl] for n in names}
    split_by = {n: split[n].reshape((b,) + tuple(shapes[n])) for n in names}
    if cfg.use_1d_linf_input_restriction_patch and b == 1:
        sub = _restrict_1d_linf(module, sub, {n: v[0] for n, v in split_by.items()})
        if sub is None:
            return {"closed": [True], "node_lower": [0.0], "node_upper": [0.0], "branch_layer": [-1],
                    "branch_neuron": [0], "split": split, "alpha": {}, "beta": {}}
    C = None if linear_spec_C is None else linear_spec_C[ex]
    warm_a = {n: front.alpha[n][sl].reshape((b,) + tuple(shapes[n])) for n in names}
    warm_b = {n: front.beta[n][sl].reshape((b,) + tuple(shapes[n])) for n in names}
    ab = cfg.oracle == "alpha_beta"
    prune = ab and b > 1 and bool(cfg.enable_batch_infeasible_prune)
    # the certificate where its verdict is known to be needed (a lone node, or pre-pruning)
    cert = split_certificate(module, sub, split_by, shapes) if ab and (b == 1 or prune) else None
    trace = forward_ibp_trace(module, sub, relu_split_state=split_by, chain=chain, raise_on_infeasible=False,
                              relu_inputs_only=True)
    layer, neuron, _gap = branch_tensors(trace, b)
    if ab:
        bounds, alpha, beta, _stats = run_alpha_beta_crown_mlp(
            module, sub, linear_spec_C=C, relu_split_state=split_by, steps=int(cfg.alpha_steps),
            lr=float(cfg.alpha_lr), alpha_init=float(cfg.alpha_init), beta_init=float(cfg.beta_init),
            warm_start_alpha=warm_a, warm_start_beta=warm_b, per_batch_params=True, trace=trace,
            first_layer_certificate=False, **_objective_kw(cfg))
    else:
        # alpha oracle: one node per round, shared alpha of that node, no split multipliers
        bounds, alpha, _stats = run_alpha_crown_mlp(
            module, sub, linear_spec_C=C, steps=int(cfg.alpha_steps), lr=float(cfg.alpha_lr),
            alpha_init=float(cfg.alpha_init), warm_start={n: v[0] for n, v in warm_a.items()},
            relu_split_state=split_by, trace=trace, **_objective_kw(cfg))
        alpha = {n: v.reshape((1,) + tuple(v.shape)) for n, v in alpha.items()}
        beta = warm_b
    rows = [bounds.lower.min(dim=1).values.double(), bounds.upper.max(dim=1).values.double(),
            trace.infeasible.double(), layer.double(), neuron.double()]
    if cert is not None:
        rows.append(cert.double())
    summary = torch.stack(rows).cpu().tolist()
    lo, up, inf, lay, neu = summary[:5]
    ibp_inf = [v != 0 for v in inf]
    cert_h = None
    if cert is not None:
        cert_h = [int(v) for v in summary[5]]
        check_flags(cert_h)
    if b == 1:
        closed = [ibp_inf[0] or (cert_h is not None and cert_h[0] == 1)]
    else:
        pruned = [prune and cert_h[i] == 1 for i in range(b)]
        rest = [i for i in range(b) if not pruned[i]]
        if any(ibp_inf[i] for i in rest):
            # the reference's batched call raises; it evaluates every remaining node alone,
            # each behind the certificate
            if cert_h is None:
                cert_h = [int(v) for v in split_certificate(module, sub, split_by, shapes).cpu().tolist()]
                check_flags(cert_h)
            closed = [pruned[i] or ibp_inf[i] or cert_h[i] == 1 for i in range(b)]
        else:
            closed = pruned
    return {"closed": closed, "node_lower": lo, "node_upper": up,
            "branch_layer": [int(v) for v in lay], "branch_neuron": [int(v) for v in neu],
            "split": split, "alpha": {n: v.reshape(b, -1) for n, v in alpha.items()},
            "beta": {n: v.reshape(b, -1) for n, v in beta.items()}}


def _restrict_1d_linf(module, spec: InputSpec, split: Dict[str, torch.Tensor]) -> Optional[InputSpec]:
    """The reference's 1-D input restriction (bab.py:524-628): a one-input Linf
    spec of one node narrowed to the interval where every first-layer split
    s * (w_i x + b_i) >= 0 of a linear layer reading the input holds; None when
    the interval is empty.  Any other spec is returned unchanged.  Scalar host
    arithmetic in Python floats, as the reference's."""
    if spec.center.dim() != 2 or int(spec.center.shape[1]) != 1 or int(spec.center.shape[0]) != 1:
        return spec
    p = spec.perturbation
    if not isinstance(p, LpBallPerturbation) or p.normalized_p() != "inf":
        return spec
    task = module.get_entry_task()
    params = module.params
    x0 = float(spec.center[0, 0].item())
    eps = float(p.eps)
    lo, hi = x0 - eps, x0 + eps
    for op in task.ops:
        if op.op_type != "relu" or op.inputs[0] not in split:
            continue
        x = op.inputs[0]
        prod = next((q for q in task.ops if x in q.outputs), None)
        if prod is None or prod.op_type != "linear" or not prod.inputs or prod.inputs[0] != spec.value_name:
            continue
        W = params.get(prod.inputs[1])
        if W is None or W.dim() != 2 or int(W.shape[1]) != 1:
            continue
        if len(prod.inputs) == 3:
            bb = params.get(prod.inputs[2])
            if bb is None or bb.dim() != 1 or int(bb.shape[0]) != int(W.shape[0]):
                continue
            b_h = bb.detach().cpu().tolist()
        else:
            b_h = [0.0] * int(W.shape[0])
        w_h = W.detach().cpu().reshape(-1).tolist()
        s_h = split[x].detach().cpu().reshape(-1).tolist()
        for i, sg in enumerate(s_h):
            if sg == 0:
                continue
            wi, bi = float(w_h[i]), float(b_h[i])
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
    center = torch.tensor([[0.5 * (lo + hi)]], device=spec.center.device, dtype=spec.center.dtype)
    return InputSpec.linf(value_name=spec.value_name, center=center, eps=float(0.5 * (hi - lo)))


# ---------------------------------------------------------------------------
# The native ReLU-split queue (boundflow/runtime/native_relu_split_bab_runtime.py:592-789)


@dataclass(frozen=True)
class NativeReluSplitBabConfig:
    """Queue and node-batching policy, field for field as the reference's
    (native_relu_split_bab_runtime.py:61-97)."""

    max_nodes: int
    max_depth: int
    expansion_batch_size: int
    max_eval_batch_size: int
    threshold: float = 0.0
    available_memory_bytes: int = 1 << 30
    memory_budget_bytes: int = 1 << 30

    def validate(self) -> None:
        if (self.max_nodes < 1 or self.max_depth < 0 or self.expansion_batch_size < 1
                or self.max_eval_batch_size < 1 or self.available_memory_bytes < 1 or self.memory_budget_bytes < 1
                or self.memory_budget_bytes > self.available_memory_bytes):
            raise ValueError("native ReLU-split BaB config is invalid")
        if not torch.isfinite(torch.tensor(self.threshold)):
            raise ValueError("native ReLU-split BaB threshold must be finite")


@dataclass(frozen=True)
class ReluSplitBranch:
    relu_input: str
    neuron_index: int
    lower: float
    upper: float
    width: float


@dataclass(frozen=True)
class NativeReluSplitBabEvaluation:
    node_id: str
    parent_node_id: Optional[str]
    depth: int
    branch_relu_input: Optional[str]
    branch_neuron_index: Optional[int]
    branch_value: int
    lower: float
    upper: float
    priority: float
    eval_batch_id: str
    eval_batch_position: int
    branch_candidate: Optional[ReluSplitBranch]


@dataclass(frozen=True)
class NativeReluSplitBabDecision:
    decision_index: int
    node_id: str
    kind: str                       # "prune" | "expand" | "terminal"
    reason: str
    child_node_ids: Tuple[str, ...] = ()
    branch_candidate: Optional[ReluSplitBranch] = None


@dataclass(frozen=True)
class NativeReluSplitBabTrace:
    run_id: str
    status: str                     # "complete" | "budget_exhausted"
    termination_reason: str
    config: NativeReluSplitBabConfig
    evaluations: Tuple[NativeReluSplitBabEvaluation, ...]
    decisions: Tuple[NativeReluSplitBabDecision, ...]
    final_frontier_node_ids: Tuple[str, ...]
    native_stack_count: int
    max_queue_size: int


def native_priority(lower: float) -> float:
    """The queue key of a node (native_relu_split_bab_runtime.py:1128-1131): its lower
    bound to 7 significant digits, so near-equal bounds fall back to creation order."""
    if not math.isfinite(lower):
        raise ValueError("native ReLU-split queue bound must be finite")
    return float(f"{lower:.7g}")


def run_native_relu_split_bab(module, input_spec, *, linear_spec_C: torch.Tensor, run_id: str,
                              config: NativeReluSplitBabConfig) -> NativeReluSplitBabTrace:
    """HIP counterpart of run_native_relu_split_bab (native_relu_split_bab_runtime.py:592-789):
    a bounded best-first queue over one box input and one scalar objective.

    Node bound: CROWN with the ADAPTIVE lower slope (``bf_alpha_adaptive``) over
    the node's IBP trace with its splits applied, on the box repeated per node,
    in batches of at most ``max_eval_batch_size`` nodes (the root, then each
    round's children).  Branch: the widest unsplit ambiguous neuron, width in
    double, ties to the first ReLU name in sorted order then the lowest index
    (``bf_branch_update_native``).  A round pops up to ``expansion_batch_size``
    queue entries (priority, serial, node id) and prunes (lower >= threshold),
    stops at the depth limit or without a branch, stops the search when two more
    nodes would pass ``max_nodes`` (the round's remaining entries return to the
    queue), or expands into the inactive then active child.  Split vectors stay
    on the device; each evaluated batch returns its bounds and branches in one
    transfer.  An infeasible split raises ValueError, as in the reference."""
    if not run_id:
        raise ValueError("native ReLU-split BaB run ID must be non-empty")
    config.validate()
    module.validate()
    spec = normalize_input_spec(input_spec)
    if not isinstance(spec.perturbation, BoxPerturbation):
        raise NotImplementedError("native ReLU-split BaB v1 requires a box input")
    lo0, hi0 = spec.perturbation.lower, spec.perturbation.upper
    if int(lo0.shape[0]) != 1:
        raise ValueError("native ReLU-split BaB v1 requires one root domain")
    C = linear_spec_C.detach()
    if C.dim() == 3:
        if int(C.shape[0]) != 1:
            raise ValueError("native ReLU-split objective batch must be one")
        C = C[0]
    if C.dim() != 2 or int(C.shape[0]) != 1:
        raise ValueError("native ReLU-split v1 requires one scalar objective")
    chain, relu_shapes, _has_conv = _relu_layout(module, spec)
    names = sorted(relu_shapes)
    if not names:
        raise ValueError("native ReLU-split BaB requires at least one ReLU")
    sizes = {n: int(torch.tensor(relu_shapes[n]).prod()) for n in names}
    dev = spec.center.device
    front = _Frontier(sizes, dev, capacity=max(64, 2 * int(config.max_eval_batch_size)))
    stream = _lib.stream_handle()
    meta: Dict[str, dict] = {}       # node id -> lineage, slot, results
    evaluations: List[NativeReluSplitBabEvaluation] = []
    decisions: List[NativeReluSplitBabDecision] = []
    counters = {"batches": 0, "next": 1}

    def evaluate(node_ids: List[str]) -> None:
        for start in range(0, len(node_ids), int(config.max_eval_batch_size)):
            chunk = node_ids[start:start + int(config.max_eval_batch_size)]
            k = len(chunk)
            batch_id = f"{run_id}:eval:{counters['batches']:04d}"
            counters["batches"] += 1
            sl = torch.tensor([meta[n]["slot"] for n in chunk], device=dev, dtype=torch.long)
            split_by = {n: front.split[n][sl].reshape((k,) + tuple(relu_shapes[n])) for n in names}
            rep = (k,) + (1,) * (lo0.dim() - 1)
            bspec = InputSpec.box(value_name=spec.value_name, lower=lo0.repeat(rep), upper=hi0.repeat(rep))
            trace = forward_ibp_trace(module, bspec, relu_split_state=split_by, chain=chain, relu_inputs_only=True)
            alpha = {}
            for n, pre in trace.relu_pre.items():
                a = torch.empty_like(pre.lower)
                _lib.call("bf_alpha_adaptive", _lib.ptr(pre.lower), _lib.ptr(pre.upper), pre.lower.numel(),
                          _lib.ptr(a), stream)
                alpha[n] = a
            Ck = C.unsqueeze(0).expand(k, -1, -1).contiguous()
            if chain is not None:
                from .crown import crown_backward
                bounds = crown_backward(module, bspec, trace, chain=chain, linear_spec_C=Ck, relu_alpha=alpha)
            else:
                from .crown_dag import crown_backward_dag
                bounds = crown_backward_dag(module, bspec, trace, linear_spec_C=Ck, relu_alpha=alpha)
            width = torch.full((k,), -1.0, device=dev, dtype=torch.float64)
            layer = torch.full((k,), -1, device=dev, dtype=torch.int32)
            idx = torch.zeros(k, device=dev, dtype=torch.int32)
            blo = torch.zeros(k, device=dev)
            bhi = torch.zeros(k, device=dev)
            for li, n in enumerate(names):
                pre = trace.relu_pre[n]
                _lib.call("bf_branch_update_native", _lib.ptr(pre.lower.reshape(k, sizes[n])),
                          _lib.ptr(pre.upper.reshape(k, sizes[n])), _lib.ptr(split_by[n].reshape(k, sizes[n])),
                          sizes[n], k, sizes[n], li, _lib.ptr(width), _lib.ptr(layer), _lib.ptr(idx), _lib.ptr(blo),
                          _lib.ptr(bhi), stream)
            rows = torch.stack([bounds.lower[:, 0].double(), bounds.upper[:, 0].double(), layer.double(),
                                idx.double(), blo.double(), bhi.double(), width]).cpu().tolist()
            for j, nid in enumerate(chunk):
                m = meta[nid]
                lay = int(rows[2][j])
                branch = None if lay < 0 else ReluSplitBranch(names[lay], int(rows[3][j]), rows[4][j], rows[5][j],
                                                              rows[6][j])
                m.update(lower=rows[0][j], upper=rows[1][j], branch=branch, priority=native_priority(rows[0][j]))
                evaluations.append(NativeReluSplitBabEvaluation(
                    node_id=nid, parent_node_id=m["parent"], depth=m["depth"], branch_relu_input=m["via"][0],
                    branch_neuron_index=m["via"][1], branch_value=m["via"][2], lower=m["lower"], upper=m["upper"],
                    priority=m["priority"], eval_batch_id=batch_id, eval_batch_position=j, branch_candidate=branch))

    root_id = f"{run_id}:n000000"
    root_slot = front.alloc(1)[0]
    for n in names:
        front.split[n][root_slot].zero_()
    meta[root_id] = {"slot": root_slot, "parent": None, "depth": 0, "via": (None, None, 0)}
    evaluate([root_id])
    heap: List[Tuple[float, int, str]] = [(meta[root_id]["priority"], 0, root_id)]
    max_q = 1
    exhausted = False
    while heap and not exhausted:
        selected = [heapq.heappop(heap) for _ in range(min(int(config.expansion_batch_size), len(heap)))]
        generated: List[str] = []
        n_dec = len(decisions)
        for pos, entry in enumerate(selected):
            nid = entry[2]
            m = meta[nid]
            if m["lower"] >= float(config.threshold):
                decisions.append(NativeReluSplitBabDecision(len(decisions), nid, "prune",
                                                            "lower_bound_meets_threshold"))
                continue
            if m["depth"] >= int(config.max_depth):
                decisions.append(NativeReluSplitBabDecision(len(decisions), nid, "terminal", "configured_depth_limit"))
                continue
            br = m["branch"]
            if br is None:
                decisions.append(NativeReluSplitBabDecision(len(decisions), nid, "terminal",
                                                            "no_unsplit_ambiguous_relu"))
                continue
            if len(evaluations) + len(generated) + 2 > int(config.max_nodes):
                for pending in selected[pos:]:
                    heapq.heappush(heap, pending)
                exhausted = True
                break
            kids = []
            slots = front.alloc(2)
            src = torch.tensor([m["slot"], m["slot"]], device=dev, dtype=torch.long)
            dst = torch.tensor(slots, device=dev, dtype=torch.long)
            for n in names:
                front.split[n][dst] = front.split[n][src]
            for side, (val, slot) in enumerate(zip((-1, 1), slots)):
                front.split[br.relu_input][slot, br.neuron_index] = val
                kid = f"{run_id}:n{counters['next']:06d}"
                counters["next"] += 1
                meta[kid] = {"slot": slot, "parent": nid, "depth": m["depth"] + 1,
                             "via": (br.relu_input, br.neuron_index, val)}
                kids.append(kid)
            generated.extend(kids)
            decisions.append(NativeReluSplitBabDecision(len(decisions), nid, "expand",
                                                        "widest_unsplit_ambiguous_relu", tuple(kids), br))
        if generated:
            evaluate(generated)
            for kid in generated:
                heapq.heappush(heap, (meta[kid]["priority"], counters["next"], kid))
            max_q = max(max_q, len(heap))
        # nodes decided this round left the queue for good: their split rows are reused
        # (the children's copies are ordered before any later write on the stream)
        front.release([meta[d.node_id]["slot"] for d in decisions[n_dec:]])
    frontier = tuple(e[2] for e in sorted(heap, key=lambda e: (e[0], e[1])))
    return NativeReluSplitBabTrace(
        run_id=run_id, status="budget_exhausted" if exhausted else "complete",
        termination_reason="node_budget_exhausted" if exhausted else "configured_bounded_tree_exhausted",
        config=config, evaluations=tuple(evaluations), decisions=tuple(decisions), final_frontier_node_ids=frontier,
        native_stack_count=counters["batches"], max_queue_size=max_q)
