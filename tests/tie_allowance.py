"""Tie allowances of the alpha / beta gradients of a CROWN lower bound (test
infrastructure; float64, on the CPU).

The lower bound is piecewise smooth in alpha and beta: it has kinks where a
coefficient changes sign.  Two correct fp32 computations that sum in different
orders can land on different sides of a kink when the coefficient there is
within rounding of zero, and their gradients then differ by a jump (a valid
subgradient each).  Two kinds:

* an input-layer coefficient y (the Linf concretization's eps * |y| term): the
  gradient dL/dy jumps by 2 * eps * |G|;
* a coefficient A entering a ReLU relaxation (the slope select A >= 0 picks the
  lower or the upper line): dL/dA jumps by |go (alpha_l - alpha_u) + G (beta_l - beta_u)|
  with go the gradient of the relaxed coefficient.

A jump dJ at an element e moves dL/dtheta by at most dJ * |de/dtheta|, so the
allowance of theta sums that over the elements that are within ``slack`` times
their fp32 rounding error of zero, the first-order effect of each tie decided
the other way.  The rounding error is the probabilistic estimate of a chain of
contractions (Higham and Mary, 2019): a length-n sum rounds by about
sqrt(n) u sum |a_i w_i| (u = 2^-24), errors already in A add in quadrature
through W, and a relaxation scales them by its slope.  (The worst-case bound
n u |A| |W| + err |W| grows with |W|'s column sums at every layer and marks
most input coefficients of a four-layer network as ties.)
Restated for chain MLPs (linear / relu) with an Linf input and per-domain
parameters, mirroring the oracle's dense equations (oracle/crown_ref.py
relu_backward_dense); domains do not interact, so callers pass only the
domains whose gradients need explaining."""

from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from oracle import alpha_beta_ref as ab
from oracle import crown_ref as cr


def tie_allowances(w64, alpha64: Dict[str, torch.Tensor], beta64: Optional[Dict[str, torch.Tensor]], splits,
                   *, slack: float = 4.0):
    """(alpha allowances, beta allowances, number of ties) of L = -sum_d mean_s lb."""
    module, spec = w64.module, w64.spec
    params = module.params
    ops = module.get_entry_task().ops
    lin = [op for op in ops if op.op_type == "linear"]
    relus = [op for op in ops if op.op_type == "relu"]
    if len(lin) != len(relus) + 1 or any(op.op_type not in ("linear", "relu") for op in ops):
        raise NotImplementedError("tie allowances are restated for chain MLPs")
    _env, pre = cr.forward_ibp_trace(module, spec, relu_split_state=splits)
    B = int(spec.center.shape[0])
    C = w64.C.double()
    S = int(C.shape[1])
    u32 = 2.0 ** -24
    a = {k: v.clone().requires_grad_(True) for k, v in alpha64.items()}
    bt = None if beta64 is None else {k: v.clone().requires_grad_(True) for k, v in beta64.items()}
    add = ab.beta_to_pre_add(bt, pre, splits) if bt is not None else {}
    A = C
    err = torch.zeros_like(C)
    b = torch.zeros(B, S, dtype=torch.float64)
    kinks = []
    for i in reversed(range(len(lin))):
        W = params[lin[i].inputs[1]].double()
        if len(lin[i].inputs) == 3:
            b = b + (A * params[lin[i].inputs[2]].double()).sum(-1)
        n = int(W.shape[0])
        err = (n ** 0.5) * u32 * (A.detach().abs() @ W.abs()) + ((err * err) @ (W * W)).sqrt()
        A = A @ W
        if i == 0:
            break
        name = relus[i - 1].inputs[0]
        _pf, au, bu, al, bl = cr.relu_backward_relaxation(pre[name], name, a)
        nn = A >= 0
        sel_a = torch.where(nn, al.unsqueeze(1), au.unsqueeze(1))
        sel_b = torch.where(nn, bl.unsqueeze(1), bu.unsqueeze(1))
        b = b + (A * sel_b).sum(-1)
        Ap = A * sel_a
        if name in add:
            Ap = Ap + cr.broadcast_pre_add(add[name], B, int(A.shape[2])).unsqueeze(1)
        Ap.retain_grad()
        kinks.append((A, err, Ap, (al - au).detach(), (bl - bu).detach()))
        err = err * torch.maximum(al.abs(), au.abs()).detach().unsqueeze(1) + u32 * Ap.detach().abs()
        A = Ap
    eps = float(spec.perturbation.eps)
    x0 = spec.center.double().reshape(B, 1, -1)
    lb = (A * x0).sum(-1) - eps * A.abs().sum(-1) + b
    loss = -lb.mean(dim=1).sum()
    loss.backward(retain_graph=True)
    G = torch.full((B, S), -1.0 / S, dtype=torch.float64)
    plist = list(a.items()) + ([] if bt is None else [(("beta", k), v) for k, v in bt.items()])
    allow = {k: torch.zeros_like(v) for k, v in plist}
    count = 0

    def accumulate(elem, jump):
        grads = torch.autograd.grad(elem, [v for _k, v in plist], retain_graph=True, allow_unused=True)
        for (k, _v), g in zip(plist, grads):
            if g is not None:
                allow[k] += jump * g.abs()

    # input-layer coefficients within rounding of zero
    for d, s, j in (A.detach().abs() <= slack * err).nonzero().tolist():
        accumulate(A[d, s, j], 2.0 * eps * abs(float(G[d, s])))
        count += 1
    # relaxation selects within rounding of zero
    for Ak, ek, Apk, dal, dbl in kinks:
        go = Apk.grad
        for d, s, n in (Ak.detach().abs() <= slack * ek).nonzero().tolist():
            jump = abs(float(go[d, s, n] * dal[d, n] + G[d, s] * dbl[d, n]))
            if jump > 0.0:
                accumulate(Ak[d, s, n], jump)
                count += 1
    allow_a = {k: allow[k].detach() for k in a}
    allow_b = {} if bt is None else {k: allow[("beta", k)].detach() for k in bt}
    return allow_a, allow_b, count
