"""Tracing the alpha / alpha-beta optimisation trajectories of the HIP path
against the CPU oracle (test infrastructure: only tests/ and bench.py's parity
leg use it; float64 checks on the CPU).

An Adam trajectory is not a continuous function of fp32 rounding: Adam divides
every element's step by the root of that element's own gradient history, so an
element whose gradient is small next to the tensor's largest (its fp32
uncertainty, 1e-6 of the gradient's scale, is a large share of it), near zero,
or at a kink of the bound (a coefficient within rounding of zero picks the
slope or the |.| sign) takes a step whose size or sign is decided by rounding.
Two correct fp32 runs then leave each other, and their best-of bounds can end
outside the 1e-5 / 1e-6 bound contract.  Instead of a band around the whole
trajectory, two checks pin every step of it:

* ``shadow_check``: along the HIP path's OWN trajectory (the states it recorded,
  ``record=``), at every step, the oracle is evaluated at the HIP state in fp32
  and fp64.  Every HIP lower bound and gradient element must be within its fp32
  uncertainty of the fp64 value: twice the larger of the contract (absolute
  1e-6 + 1e-5 relative for bounds; 1e-6 of the gradient's scale + 1e-5 relative
  for gradients) and the oracle's own fp32 error -- where one run does not
  explain a value, the largest error over the oracle run and REORDERINGS runs of
  the same network with its units permuted (other summation orders: one fp32
  run is one sample of the rounding) -- or, for gradients, inside the computed
  kink allowance of oracle/gradients.py; the HIP
  parameters after the step must equal torch's fp32 Adam (and the clamp) applied
  to the HIP gradient with moments rebuilt on the CPU from the HIP gradient
  history.  The final best-of bounds must be one of the recorded evaluations
  with the best metric.  So every step the HIP path takes is a step of the
  reference algorithm up to fp32 rounding.
* ``divergence_trace``: for every domain whose final bounds leave the contract,
  the first step k* at which the HIP and oracle parameters part (outside the
  contract), the elements that part, and why.  The HIP value after k* must lie
  in the set Adam reaches from the ORACLE's state when each gradient of the
  history 0..k* moves within its uncertainty radius -- computed from the oracle
  alone (fp32 vs fp64 at the oracle state, the fp64 gradient's change between
  the two states, the contract on the gradient's scale and any kink allowance),
  never from the HIP gradient -- and so must the oracle's own value.  Each
  element is classified: "sign" (the radius at k* reaches zero: the gradient's
  sign is not decided in fp32), "kink" (a kink allowance was needed on the
  history), or "normalisation" (a small element whose relative uncertainty Adam's
  per-element normalisation turns into a step difference).

Reference: the optimisation loop of alpha_beta_crown.py:756-925 (Adam over alpha
and beta, clamps, best-of over steps + 1 evaluations)."""

from __future__ import annotations

from typing import Dict, List, Optional

import torch

from oracle import parity
from oracle.gradients import oracle_grads, permuted_oracle_grads, tie_allowances_for_domains

RTOL, ATOL = 1e-5, 1e-6
B1, B2, EPS = 0.9, 0.999, 1e-8


def _stderr(msg: str) -> None:
    import sys
    print(msg, file=sys.stderr, flush=True)


def sub_workload(w, idx: torch.Tensor):
    """The domains ``idx`` of a workload (same network; splits sliced too)."""
    from boundflow_amd import workloads as wl
    from boundflow_amd.spec import BoxPerturbation, InputSpec
    p = w.spec.perturbation
    if isinstance(p, BoxPerturbation):
        spec = InputSpec.box(value_name=w.spec.value_name, lower=p.lower[idx], upper=p.upper[idx])
    else:
        spec = InputSpec(value_name=w.spec.value_name, center=w.spec.center[idx], perturbation=p)
    extra = {}
    if "splits" in w.extra:
        extra["splits"] = {k: v[idx] for k, v in w.extra["splits"].items()}
    return wl.Workload(w.name, w.module, spec, w.C[idx], w.labels[idx], extra)


def slice_record(rec: List[dict], idx: torch.Tensor) -> List[dict]:
    """Per-domain slice of a recorded trajectory (oracle or HIP ``record=`` lists)."""
    out = []
    for r in rec:
        s = {}
        for key, val in r.items():
            if isinstance(val, dict):
                s[key] = {k: (None if v is None else v[idx]) for k, v in val.items()}
            elif isinstance(val, torch.Tensor) and val.dim() > 0:
                s[key] = val[idx]
            else:
                s[key] = val
        out.append(s)
    return out


def outside(got: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    g, r = got.double(), ref.double()
    return (g - r).abs() > ATOL + RTOL * r.abs()


def domains_outside(got: torch.Tensor, ref: torch.Tensor) -> List[int]:
    """Rows (domains) with any bound outside the contract."""
    return outside(got, ref).reshape(got.shape[0], -1).any(dim=1).nonzero().flatten().tolist()


def _flat(t: torch.Tensor, B: int) -> torch.Tensor:
    return t.reshape(B, -1).double()


def _params(names, beta_names):
    return [("alpha", n) for n in names] + [("beta", n) for n in beta_names]


def _oracle_at(w, alpha, beta, splits, dtype):
    """(lower, {(kind, name): gradient [B, n]}) of L = -sum_d mean_s lb at (alpha, beta)."""
    B = int(w.C.shape[0])
    b, ga, gb = oracle_grads(w, alpha, beta, splits, dtype=dtype)
    g = {("alpha", k): _flat(v, B) for k, v in ga.items()}
    if beta is not None:
        for k, v in beta.items():
            got = None if gb is None else gb.get(k)
            g[("beta", k)] = torch.zeros_like(_flat(v, B)) if got is None else _flat(got, B)
    return b.lower, g


def bounds_at(w, alpha: Dict[str, torch.Tensor], dtype=torch.float32):
    """The oracle's (lower, upper) bounds of ``w`` at per-domain slopes ``alpha`` and no
    split multipliers (the reference's final upper-bound evaluation, which takes the
    best alpha and no beta, alpha_beta_crown.py:763-785)."""
    from oracle import crown_ref as cr
    if dtype == torch.float64:
        w = parity.to_float64(w)
    a = {k: v.to(dtype) for k, v in alpha.items()}
    env, pre = cr.forward_ibp_trace(w.module, w.spec, relu_split_state=w.extra.get("splits"))
    b = cr.crown_backward_from_trace(w.module, w.spec, interval_env=env, relu_pre=pre, linear_spec_C=w.C,
                                     relu_alpha=a)
    return b.lower.detach(), b.upper.detach()


# summation orders sampled (besides the oracle's own) where one fp32 run does not explain a value
REORDERINGS = 4


def _tolerance(g32: torch.Tensor, g64: torch.Tensor, scale: Optional[float] = None) -> torch.Tensor:
    """fp32 uncertainty radius of a tensor around its fp64 value: twice the larger of the
    oracle's own fp32 error and the contract -- on the gradient's scale (the tensor's
    largest magnitude) for gradients, or absolute (``scale=0.0``: 1e-6) for bounds."""
    g32, g64 = g32.double(), g64.double()
    floor = ATOL * ((float(g64.abs().max()) + 1e-30) if scale is None else 1.0)
    return 2.0 * torch.maximum((g32 - g64).abs(), floor + RTOL * g64.abs())


def _adam_replay(p, g, m, v, t, lr, lo, hi):
    """torch.optim.Adam (fp32, CPU) one step from moments (m, v) at step t, then the clamp;
    returns (new parameter, new m, new v)."""
    q = p.detach().float().clone().requires_grad_(True)
    opt = torch.optim.Adam([q], lr=lr)
    st = {"step": torch.tensor(float(t - 1)), "exp_avg": m.float().clone(), "exp_avg_sq": v.float().clone()}
    opt.state[q] = st
    q.grad = g.float().clone()
    opt.step()
    with torch.no_grad():
        q.clamp_(lo, hi) if hi is not None else q.clamp_(min=lo)
    return q.detach(), opt.state[q]["exp_avg"].clone(), opt.state[q]["exp_avg_sq"].clone()


def adam_reach(p: torch.Tensor, centers: List[torch.Tensor], radii: List[torch.Tensor], lr: float, lo: float,
               hi: Optional[float]):
    """[lo, hi] enclosure of the clamped Adam parameter after len(centers) steps'
    moments, taken from parameter value p at the last step, when gradient j of the
    history lies anywhere in [centers[j] - radii[j], centers[j] + radii[j]] (float64,
    elementwise).  m and v are enclosed separately (m linear, v a sum of squares);
    the normalised step m / sqrt(v) is further bounded by Cauchy-Schwarz,
    |m| <= sqrt(sum c_j^2 / d_j) sqrt(v), with c_j, d_j the moments' weights."""
    t = len(centers)
    m_lo = torch.zeros_like(p)
    m_hi = torch.zeros_like(p)
    v_lo = torch.zeros_like(p)
    v_hi = torch.zeros_like(p)
    for c, r in zip(centers, radii):
        a, b = c - r, c + r
        m_lo = B1 * m_lo + (1.0 - B1) * a
        m_hi = B1 * m_hi + (1.0 - B1) * b
        sq_lo = torch.where((a <= 0) & (b >= 0), torch.zeros_like(a), torch.minimum(a * a, b * b))
        v_lo = B2 * v_lo + (1.0 - B2) * sq_lo
        v_hi = B2 * v_hi + (1.0 - B2) * torch.maximum(a * a, b * b)
    bc1, bc2 = 1.0 - B1 ** t, 1.0 - B2 ** t
    sb = bc2 ** 0.5
    cs = sum(((1.0 - B1) * B1 ** (t - 1 - j)) ** 2 / ((1.0 - B2) * B2 ** (t - 1 - j)) for j in range(t)) ** 0.5
    R = cs * sb
    den_lo = v_lo.sqrt() / sb + EPS
    den_hi = v_hi.sqrt() / sb + EPS
    f_hi = torch.where(m_hi > 0, m_hi / den_lo, m_hi / den_hi).clamp(-R, R)
    f_lo = torch.where(m_lo < 0, m_lo / den_lo, m_lo / den_hi).clamp(-R, R)
    step = lr / bc1
    out_lo, out_hi = p - step * f_hi, p - step * f_lo
    if hi is not None:
        return out_lo.clamp(lo, hi), out_hi.clamp(lo, hi)
    return out_lo.clamp(min=lo), out_hi.clamp(min=lo)


class ShadowResult:
    def __init__(self):
        self.g64: List[Dict] = []       # per step: {(kind, name): fp64 gradient at the HIP state}
        self.tol: List[Dict] = []       # per step: uncertainty radius at the HIP state (allowance included)
        self.allow: List[Dict] = []     # per step: the kink allowance part of it (zero where none)
        self.ties = 0
        self.reordered = 0              # domain-steps whose radius took the spread over summation orders


def shadow_check(w, hrec: List[dict], lr: float, names: List[str], beta_names: List[str], what: str,
                 final_lower: Optional[torch.Tensor] = None, log=_stderr) -> ShadowResult:
    """Along the HIP path's own trajectory ``hrec`` (domains of ``w``), every step: bounds
    at the contract against the oracle at the HIP state, gradients within their fp32
    uncertainty (or a computed kink allowance), the Adam update reproduced by torch's fp32
    Adam from the HIP gradient and the rebuilt moments.  ``final_lower``: the HIP best-of
    lower bound, which must equal a recorded evaluation with the best metric."""
    splits = w.extra.get("splits")
    B = int(w.C.shape[0])
    res = ShadowResult()
    keys = _params(names, beta_names)
    m = {k: torch.zeros(B, _flat(hrec[0][k[0]][k[1]], B).shape[1]) for k in keys}
    v = {k: torch.zeros_like(m[k]) for k in keys}
    n_bad_bounds = 0
    for j, rec in enumerate(hrec):
        alpha = {n: rec["alpha"][n].float() for n in names}
        beta = {n: rec["beta"][n].float() for n in rec["beta"]} if beta_names else None
        lo32, g32 = _oracle_at(w, alpha, beta, splits, torch.float32)
        lo64, g64 = _oracle_at(w, alpha, beta, splits, torch.float64)
        lo32, lo64 = lo32.detach().double(), lo64.detach().double()
        lo_h = rec["lower"].double()
        lo_rad = _tolerance(lo32.double(), lo64.double(), scale=0.0)
        res.g64.append(g64)
        final = "grad_alpha" not in rec
        tol = {} if final else {k: _tolerance(g32[k], g64[k]) for k in keys}
        hip_g = {}
        if not final:
            hip_g = {("alpha", n): _flat(rec["grad_alpha"][n], B) for n in names}
            hip_g.update({("beta", n): _flat(rec["grad_beta"][n], B) for n in beta_names})

        def misses():
            lo_bad = (lo_h - lo64.double()).abs() > lo_rad
            bad = {k: (hip_g[k] - g64[k]).abs() > tol[k] for k in tol}
            rows = set(lo_bad.any(dim=1).nonzero().flatten().tolist())
            for k in tol:
                rows |= set(bad[k].any(dim=1).nonzero().flatten().tolist())
            return lo_bad, bad, sorted(rows)

        lo_bad, bad, doms = misses()
        if doms:
            # one fp32 run is one sample of the rounding: widen the radius of these domains to the
            # spread over other summation orders (the network with its units permuted)
            idx = torch.tensor(doms)
            ws = sub_workload(w, idx)
            a_s = {n: v[idx] for n, v in alpha.items()}
            b_s = None if beta is None else {n: v[idx] for n, v in beta.items()}
            spread = {k: (g32[k][idx] - g64[k][idx]).abs() for k in tol}
            lo_spread = (lo32.double()[idx] - lo64.double()[idx]).abs()
            for seed in range(1, REORDERINGS + 1):
                gp = permuted_oracle_grads(ws, a_s, b_s, ws.extra.get("splits"), seed)
                if gp is None:
                    break
                lo_spread = torch.maximum(lo_spread, (gp["lower"] - lo64.double()[idx]).abs())
                for k in tol:
                    spread[k] = torch.maximum(spread[k], (gp[k] - g64[k][idx]).abs())
            for k in tol:
                tol[k][idx] = torch.maximum(tol[k][idx], 2.0 * spread[k])
            lo_rad[idx] = torch.maximum(lo_rad[idx], 2.0 * lo_spread)
            res.reordered += len(doms)
            lo_bad, bad, doms = misses()
        if bool(lo_bad.any()):
            d, s_ = lo_bad.nonzero()[0].tolist()
            log(f"{what} step {j} lower at the HIP state: {int(lo_bad.sum())} values outside the fp32 spread, e.g. "
                f"domain {d} spec {s_}: hip {float(lo_h[d, s_])} fp32 {float(lo32[d, s_])} fp64 {float(lo64[d, s_])} "
                f"radius {float(lo_rad[d, s_])}")
        n_bad_bounds += int(lo_bad.sum())
        if final:
            res.tol.append({})
            res.allow.append({})
            continue
        doms = sorted({d for k in keys for d in bad[k].any(dim=1).nonzero().flatten().tolist()})
        allowed = {k: torch.zeros_like(tol[k]) for k in keys}
        if doms:
            allow, _nt = tie_allowances_for_domains(w, {"alpha": alpha, "beta": beta or {}}, splits, doms,
                                                    bool(beta_names))
            for k in keys:
                full = torch.zeros_like(tol[k])
                full[doms] = allow[k[0]][k[1]].reshape(len(doms), -1).double()
                scale = float(g64[k].abs().max()) + 1e-30
                tol[k] = torch.maximum(tol[k], full + ATOL * scale)
                allowed[k] = full
                res.ties += int((full > 0).sum())
            bad = {k: (hip_g[k] - g64[k]).abs() > tol[k] for k in keys}
        res.tol.append(tol)
        res.allow.append(allowed)
        for k in keys:
            if bool(bad[k].any()):
                idx = bad[k].nonzero()[:4].tolist()
                detail = [(d, n, float(hip_g[k][d, n]), float(g32[k][d, n]), float(g64[k][d, n]), float(tol[k][d, n]),
                           float(allowed[k][d, n])) for d, n in idx]
                raise AssertionError(f"{what} step {j} d/d{k[0]}[{k[1]}]: {int(bad[k].sum())} elements outside their "
                                     f"fp32 uncertainty and kink allowance, e.g. (domain, element, hip, fp32, fp64, "
                                     f"radius, allowance) {detail}")
        # the Adam step: torch's fp32 Adam on the HIP gradient from the rebuilt moments
        for k in keys:
            kind, n = k
            lo, hi = (0.0, 1.0) if kind == "alpha" else (0.0, None)
            p = _flat(rec[kind][n], B)
            nxt, m[k], v[k] = _adam_replay(p, hip_g[k], m[k], v[k], j + 1, lr, lo, hi)
            got = _flat(rec[f"{kind}_next"][n], B)
            off = outside(got, nxt.double())
            if bool(off.any()):
                raise AssertionError(f"{what} step {j} Adam update of {kind}[{n}]: {int(off.sum())} elements differ "
                                     f"from torch Adam on the HIP gradient")
    assert n_bad_bounds == 0, f"{what}: {n_bad_bounds} lower bounds at HIP states outside the contract"
    if final_lower is not None:
        metrics = torch.stack([r["lower"].double().mean(dim=1) for r in hrec])       # [steps+1, B]
        best = metrics.max(dim=0).values
        near = metrics >= best - (ATOL + RTOL * best.abs())
        fl = final_lower.double()
        hit = torch.stack([(r["lower"].double() == fl).all(dim=1) for r in hrec]) & near
        miss = (~hit.any(dim=0)).nonzero().flatten().tolist()
        assert not miss, f"{what}: best-of bounds of domains {miss[:8]} are no best recorded evaluation"
    log(f"{what}: shadow check over {len(hrec)} evaluations x {B} domains: bounds, gradients "
        f"({res.reordered} domain-steps on the spread over summation orders, {res.ties} kink-allowance entries) "
        f"and Adam updates at the contract")
    return res


def divergence_trace(w, hrec: List[dict], srec: List[dict], shadow: ShadowResult, lr: float, names: List[str],
                     beta_names: List[str], domains: List[int], what: str, log=_stderr) -> Dict[int, tuple]:
    """For each listed domain (rows of ``w``; both records over the same rows): the first
    step at which the HIP and oracle parameters part, checked to lie in the Adam-reachable
    enclosure built from the oracle's state and uncertainty radii; returns
    {domain: (k*, elements, categories)}."""
    splits = w.extra.get("splits")
    B = int(w.C.shape[0])
    keys = _params(names, beta_names)
    steps = len(srec) - 1
    first = {}
    for d in domains:
        k_star = -1
        for k in range(steps):
            if any(bool(outside(_flat(hrec[k][f"{kind}_next"][n], B)[d], _flat(srec[k][f"{kind}_next"][n], B)[d]).any())
                   for kind, n in keys):
                k_star = k
                break
        first[d] = k_star
    g64_s: List[Dict] = []
    out: Dict[int, tuple] = {}
    kmax = max([k for k in first.values()] + [-1])
    for j in range(kmax + 1):
        rec = srec[j]
        alpha = {n: rec["alpha"][n].float() for n in names}
        beta = {n: rec["beta"][n].float() for n in rec["beta"]} if beta_names else None
        _lo, g = _oracle_at(w, alpha, beta, splits, torch.float64)
        g64_s.append(g)
    for d in domains:
        k = first[d]
        if k < 0:
            out[d] = (-1, 0, {})
            continue
        counts = {"sign": 0, "kink": 0, "normalisation": 0}
        n_div = 0
        for kind, n in keys:
            key = (kind, n)
            h_next = _flat(hrec[k][f"{kind}_next"][n], B)[d]
            s_next = _flat(srec[k][f"{kind}_next"][n], B)[d]
            div = outside(h_next, s_next)
            if not bool(div.any()):
                continue
            n_div += int(div.sum())
            centers, radii = [], []
            used_kink = torch.zeros_like(h_next, dtype=torch.bool)
            for j in range(k + 1):
                g32 = _flat(srec[j][f"grad_{kind}"][n], B)[d] if srec[j][f"grad_{kind}"][n] is not None else \
                    torch.zeros_like(h_next)
                gs = g64_s[j][key][d]
                scale = float(g64_s[j][key].abs().max()) + 1e-30
                tol_s = 2.0 * torch.maximum((g32 - gs).abs(), ATOL * scale + RTOL * gs.abs())
                gh = shadow.g64[j][key][d]
                tol_h = shadow.tol[j][key][d]
                used_kink |= shadow.allow[j][key][d] > 0
                centers.append(gs)
                radii.append(torch.maximum(tol_s, (gh - gs).abs() + tol_h))
            lo, hi = (0.0, 1.0) if kind == "alpha" else (0.0, None)
            p_s = _flat(srec[k][kind][n], B)[d]
            p_h = _flat(hrec[k][kind][n], B)[d]
            r_lo, r_hi = adam_reach(p_s, centers, radii, lr, lo, hi)
            slack = ATOL + RTOL * s_next.abs()
            shift = (p_h - p_s).abs()
            h_in = (h_next >= r_lo - slack - shift) & (h_next <= r_hi + slack + shift)
            s_in = (s_next >= r_lo - slack) & (s_next <= r_hi + slack)
            bad = div & ~(h_in & s_in)
            if bool(bad.any()):
                e = bad.nonzero().flatten()[:4].tolist()
                raise AssertionError(f"{what} domain {d} step {k} {kind}[{n}] elements {e}: HIP "
                                     f"{h_next[e].tolist()} / oracle {s_next[e].tolist()} outside the Adam-reachable "
                                     f"range [{r_lo[e].tolist()}, {r_hi[e].tolist()}]")
            sign = div & ((centers[-1] - radii[-1]) <= 0) & ((centers[-1] + radii[-1]) >= 0)
            kink = div & ~sign & used_kink
            counts["sign"] += int(sign.sum())
            counts["kink"] += int(kink.sum())
            counts["normalisation"] += int((div & ~sign & ~kink).sum())
        out[d] = (k, n_div, counts)
    for d in domains:
        k, nd, c = out[d]
        log(f"{what} domain {d}: first divergent step {k}, {nd} parameter elements part "
                 f"(sign {c.get('sign', 0)}, kink {c.get('kink', 0)}, normalisation {c.get('normalisation', 0)}), "
                 f"all inside the Adam-reachable range of the oracle state")
    return out


def trace_run(w, hrec: List[dict], srec: List[dict], got_lower: torch.Tensor, ref_lower: torch.Tensor, lr: float, *,
              what: str, sample=(), got_upper: Optional[torch.Tensor] = None,
              ref_upper: Optional[torch.Tensor] = None, best_alpha: Optional[Dict[str, torch.Tensor]] = None,
              fp64_lower=None, log=_stderr) -> dict:
    """Whole-batch parity of an optimised bound without a trajectory band.

    ``w``: the workload over the domains both records cover (rows of every tensor
    here); ``hrec`` / ``srec``: the HIP and oracle records; ``got_*`` / ``ref_*``:
    the final best-of bounds.  Every domain with a bound outside the contract,
    plus the domains ``sample``, is shadow-checked along the HIP trajectory, and
    each out-of-contract domain's divergence is traced (both raise
    AssertionError on a failure).  A domain whose parameters never part must be
    fp64-explained: ``fp64_lower(rows)`` returns the fp64 oracle's final lower
    bound of those rows.  With ``best_alpha`` (the HIP best-of slopes, [B, ...]
    per ReLU) the HIP upper bound is checked against the oracle's upper bound at
    those slopes.  Returns a summary dict."""
    names = list(hrec[0]["alpha"].keys())
    beta_names = [n for n in names if hrec[0].get("grad_beta", {}).get(n) is not None]
    out_lo = outside(got_lower, ref_lower)
    out_doms = set(out_lo.any(dim=1).nonzero().flatten().tolist())
    n_out = int(out_lo.sum())
    if got_upper is not None and ref_upper is not None:
        out_up = outside(got_upper, ref_upper)
        out_doms |= set(out_up.any(dim=1).nonzero().flatten().tolist())
        n_out += int(out_up.sum())
    out_doms = sorted(out_doms)
    doms = sorted(set(out_doms) | set(int(d) for d in sample))
    summary = {"values_outside_contract": n_out, "domains_outside_contract": len(out_doms),
               "shadow_checked_domains": len(doms), "evaluations": len(hrec)}
    log(f"{what}: {n_out} bound values outside the contract 1e-5/1e-6 in {len(out_doms)} domains; shadow "
        f"check of {len(doms)} domains ({len(doms) - len(out_doms)} sampled in contract)")
    if not doms:
        summary.update({"first_divergent_step": {}, "divergent_elements": {}, "traced_domains": 0})
        return summary
    idx = torch.tensor(doms)
    ws = sub_workload(w, idx)
    hs, ss = slice_record(hrec, idx), slice_record(srec, idx)
    sh = shadow_check(ws, hs, lr, names, beta_names, what, final_lower=got_lower[idx], log=log)
    summary["kink_allowance_entries"] = sh.ties
    summary["reordered_domain_steps"] = sh.reordered
    if best_alpha is not None and got_upper is not None:
        a = {n: best_alpha[n][idx].float() for n in names}
        _l32, u32 = bounds_at(ws, a)
        rep = parity.compare(got_upper[idx], u32, None)
        if rep.strict_violations:
            _l64, u64 = bounds_at(ws, {n: v.double() for n, v in a.items()}, torch.float64)
            rep = parity.compare(got_upper[idx], u32, u64)
        log(rep.line(f"{what} upper at the HIP best-of slopes"))
        assert rep.ok, rep.line(f"{what} upper at the HIP best-of slopes")
    pos = [doms.index(d) for d in out_doms]
    tr = divergence_trace(ws, hs, ss, sh, lr, names, beta_names, pos, what, log=log)
    never = [doms[p] for p in pos if tr[p][0] < 0]
    if never:
        rows = torch.tensor(never)
        e = fp64_lower(rows)
        rep = parity.compare(got_lower[rows], ref_lower[rows], e)
        log(rep.line(f"{what} domains {never[:8]} whose parameters never part (fp64)"))
        assert rep.ok, f"{what}: domains {never} leave the contract with identical trajectories"
    hist: Dict[int, int] = {}
    cats = {"sign": 0, "kink": 0, "normalisation": 0}
    for p in pos:
        k, _n, c = tr[p]
        hist[k] = hist.get(k, 0) + 1
        for key in cats:
            cats[key] += int(c.get(key, 0))
    summary.update({"traced_domains": len(pos), "first_divergent_step": {str(k): v for k, v in sorted(hist.items())},
                    "divergent_elements": cats})
    return summary
