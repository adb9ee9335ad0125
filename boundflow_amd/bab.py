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

from typing import Dict, Optional

import torch

from . import _lib
from .alpha_beta import branch_tensors, run_alpha_beta_crown_mlp
from .crown import forward_ibp_trace, parse_chain
from .spec import normalize_input_spec


def evaluate_domain_batch(module, input_spec, *, linear_spec_C: torch.Tensor,
                          relu_split_state: Dict[str, torch.Tensor], steps: int = 10, lr: float = 0.2,
                          alpha_init: float = 0.5, beta_init: float = 0.0,
                          warm_start_alpha: Optional[Dict[str, torch.Tensor]] = None,
                          warm_start_beta: Optional[Dict[str, torch.Tensor]] = None,
                          threshold: float = 0.0, tol: float = 1e-6):
    """Returns a dict of device tensors: ``status`` int32 [D] (0 open, 1 certified,
    2 infeasible), ``lower``/``upper`` [D, S], ``branch_layer``/``branch_neuron``
    int32 [D] (-1 when no ambiguous neuron is left), ``alpha``/``beta`` per ReLU."""
    spec = normalize_input_spec(input_spec)
    chain = parse_chain(module, spec)
    trace = forward_ibp_trace(module, spec, relu_split_state=relu_split_state, chain=chain,
                              raise_on_infeasible=False)
    D = int(spec.center.shape[0])
    layer, neuron, _gap = branch_tensors(trace, D)
    bounds, alpha, beta, _stats = run_alpha_beta_crown_mlp(
        module, spec, linear_spec_C=linear_spec_C, relu_split_state=relu_split_state, steps=steps, lr=lr,
        alpha_init=alpha_init, beta_init=beta_init, warm_start_alpha=warm_start_alpha,
        warm_start_beta=warm_start_beta, per_batch_params=True, trace=trace)
    S = int(bounds.lower.shape[1])
    status = torch.empty(D, dtype=torch.int32, device=spec.center.device)
    _lib.call("bf_domain_status", _lib.ptr(bounds.lower), D, S, _lib.ptr(trace.infeasible), float(threshold),
              float(tol), _lib.ptr(status), _lib.stream_handle())
    return {"status": status, "lower": bounds.lower, "upper": bounds.upper, "branch_layer": layer,
            "branch_neuron": neuron, "alpha": alpha, "beta": beta, "infeasible": trace.infeasible,
            "relu_names": list(trace.relu_pre.keys())}
