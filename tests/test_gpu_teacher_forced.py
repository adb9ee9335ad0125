"""Per-step ("teacher-forced") parity of the alpha / alpha-beta optimisation at
the contract tolerance (|hip - ref| <= 1e-6 + 1e-5 |ref|).

A 20- or 10-step Adam trajectory amplifies fp32 rounding: where a gradient is
within rounding of zero, Adam's normalised step moves a parameter by up to lr
either way.  So the trajectory is not compared as a whole here; instead the
oracle's own state at a step k -- alpha_k, beta_k and Adam's moments (recorded
by ``oracle.alpha_beta_ref.run_alpha_beta_crown(record=...)``) -- is fed to the
device, and one step is compared:

* the lower bound at (alpha_k, beta_k): contract, or fp64-explained (the HIP
  value at least as close to the fp64 oracle as the fp32 reference is);
* dL/dalpha and dL/dbeta: contract on the gradient's scale, or fp64-explained,
  or inside the jump allowance of a kink: where an input-layer coefficient (its
  |.| in the concretization) or a coefficient entering a ReLU relaxation (its
  sign selects the slope) is within fp32 rounding of zero, the two fp32
  computations may take different one-sided derivatives (oracle/gradients.py);
* the Adam update: the device's clamped alpha_{k+1}, beta_{k+1} equal torch's
  fp32 Adam applied to the device's own gradient and the same moments, at the
  contract -- the optimiser step itself adds no error.  Against the oracle's
  alpha_{k+1} the elements outside the contract are counted, and each must sit
  where the exact gradient is within the two fp32 gradients' error of zero.

Configurations: C4 at its full size (B = 32, alpha from CROWN, lr 0.1) at steps
0, 1, 10, 19 and its final evaluation 20; C5's domain batch (512 domains of the
4096, 1-12 splits each, lr 0.2) at steps 0, 1, 9 and the final 10.  The
verdicts of the reference trajectory's best bounds are asserted by the
trajectory tests (tests/test_gpu_conv_alpha.py, tests/test_gpu_full_size.py)."""

import pytest
import torch

from boundflow_amd import alpha_beta as hab
from boundflow_amd import workloads as wl
from oracle import alpha_beta_ref as ab
from oracle import crown_ref as cr
from oracle import parity
from tests.gpu_util import announce, device
from oracle.gradients import oracle_grads as _oracle_grads
from oracle.gradients import tie_allowances_for_domains

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


def _trajectory(w, *, steps, lr, splits, init):
    rec = []
    ab.run_alpha_beta_crown(w.module, w.spec, linear_spec_C=w.C, relu_split_state=splits, steps=steps, lr=lr,
                            warm_start_alpha=init, per_batch_params=True, record=rec)
    return rec


def _grad_report(got, ref32, ref64, what, allowance=None):
    """Contract on the gradient's scale (atol = 1e-6 * max|g|), or fp64-explained,
    or inside the tie allowance ([B, n] or None).  Returns (HIP gradient, the
    [B, n] mask of elements left unexplained)."""
    g = got.detach().cpu().double().reshape(ref32.shape)
    r = ref32.double()
    e = ref64.double()
    scale = float(e.abs().max()) + 1e-30
    d = (g - r).abs()
    strict = d > (ATOL * scale + RTOL * r.abs())
    explained = strict & ((g - e).abs() <= 2.0 * torch.maximum((r - e).abs(), ATOL * scale + RTOL * e.abs()))
    if allowance is not None:
        explained |= strict & ((g - e).abs() <= allowance.double().reshape(g.shape) + ATOL * scale)
    bad = strict & ~explained
    announce(f"{what}: n={g.numel()} max|hip-ref|={float(d.max()):.3e} (scale {scale:.3e}) outside contract "
             f"{int(strict.sum())}, explained (fp64{'' if allowance is None else ' or ties'}) "
             f"{int(explained.sum())}, unexplained {int(bad.sum())}")
    return g, bad.reshape(g.shape[0], -1)


def _tie_allowance(w, rec, splits, doms, with_beta):
    """{"alpha": {name: [len(doms), ...]}, "beta": {...}}: the kink allowances of the
    lower bound's gradient at this step's parameters, for the listed domains."""
    allow, nt = tie_allowances_for_domains(w, rec, splits, doms, with_beta)
    announce(f"  {nt} coefficients within fp32 rounding of zero on domains {doms[:8]}")
    return allow


def _adam_ref(p, g, m, v, t, lr, lo, hi):
    """torch.optim.Adam (fp32, CPU) from the given moments, then the clamp."""
    q = p.detach().clone().requires_grad_(True)
    opt = torch.optim.Adam([q], lr=lr)
    opt.state[q] = {"step": torch.tensor(float(t - 1)), "exp_avg": m.clone(), "exp_avg_sq": v.clone()}
    q.grad = g.clone()
    opt.step()
    with torch.no_grad():
        q.clamp_(lo, hi) if hi is not None else q.clamp_(min=lo)
    return q.detach()


def _adam_range(p, g, delta, m, v, t, lr, lo, hi, samples=33):
    """[min, max] over gradients in [g - delta, g + delta] of the clamped torch Adam
    update (fp64 arithmetic) from moments m, v at step t."""
    b1, b2, eps = 0.9, 0.999, 1e-8
    bc1, bc2 = 1.0 - b1 ** t, 1.0 - b2 ** t
    out_lo = out_hi = None
    for f in torch.linspace(-1.0, 1.0, samples, dtype=torch.float64):
        gg = g + f * delta
        m2 = m + (gg - m) * (1.0 - b1)
        v2 = v * b2 + (1.0 - b2) * gg * gg
        q = p - (lr / bc1) * m2 / (v2.sqrt() / bc2 ** 0.5 + eps)
        q = q.clamp(lo, hi) if hi is not None else q.clamp(min=lo)
        out_lo = q if out_lo is None else torch.minimum(out_lo, q)
        out_hi = q if out_hi is None else torch.maximum(out_hi, q)
    return out_lo, out_hi


def _device_step(wd, rec, lr, splits_d, names, beta_names):
    """Bounds, gradients and the Adam update of one step on the device, from the oracle's state."""
    dev = wd.spec.center.device
    alpha = {k: v.to(dev).contiguous() for k, v in rec["alpha"].items()}
    beta = {k: v.to(dev).contiguous() for k, v in rec["beta"].items()} if beta_names else None
    bounds, ga, gb = hab.lower_bound_gradients(wd.module, wd.spec, linear_spec_C=wd.C, relu_alpha=alpha,
                                               relu_beta=beta, relu_split_state=splits_d, per_batch_params=True)
    params = [alpha[k].reshape(alpha[k].shape[0], -1).clone() for k in names]
    params += [beta[k].reshape(beta[k].shape[0], -1).clone() for k in beta_names]
    grads = [ga[k].reshape(params[i].shape).contiguous() for i, k in enumerate(names)]
    grads += [gb[k].reshape(params[len(names) + i].shape).contiguous() for i, k in enumerate(beta_names)]
    grp = hab._AdamGroup(params, [(0.0, 1.0)] * len(names) + [(0.0, None)] * len(beta_names))
    keys = [("alpha", k) for k in names] + [("beta", k) for k in beta_names]
    for i, key in enumerate(keys):
        grp.m[i].copy_(rec["exp_avg"][key].reshape(params[i].shape))
        grp.v[i].copy_(rec["exp_avg_sq"][key].reshape(params[i].shape))
    grp.t = int(rec["adam_step"]) - 1
    grp.step(grads, lr, hab._lib.stream_handle())
    torch.cuda.synchronize()
    return bounds, ga, gb, grp.p


def _check_step(w, wd, rec, k, lr, splits, names, beta_names):
    dev = wd.spec.center.device
    splits_d = None if splits is None else {n: v.to(dev) for n, v in splits.items()}
    has_grad = "grad_alpha" in rec
    if not has_grad:
        # the final evaluation: bounds only
        from boundflow_amd import crown as hc
        alpha = {n: v.to(dev) for n, v in rec["alpha"].items()}
        add = None
        if beta_names:
            _e, pre = cr.forward_ibp_trace(w.module, w.spec, relu_split_state=splits)
            add = {n: v.to(dev) for n, v in ab.beta_to_pre_add(rec["beta"], pre, splits).items()}
        b = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C, relu_alpha=alpha,
                                 relu_pre_add_coeff_l=add, relu_split_state=splits_d)
        ref64, _ga, _gb = _oracle_grads(w, rec["alpha"], rec["beta"] if beta_names else None, splits,
                                        dtype=torch.float64)
        rep = parity.compare(b.lower, rec["lower"], ref64.lower)
        announce(rep.line(f"step {k} lower (final evaluation)"))
        assert rep.ok
        return
    bounds, ga, gb, new_params = _device_step(wd, rec, lr, splits_d, names, beta_names)
    ref64, ga64, gb64 = _oracle_grads(w, rec["alpha"], rec["beta"] if beta_names else None, splits,
                                      dtype=torch.float64)
    rep = parity.compare(bounds.lower, rec["lower"], ref64.lower)
    announce(rep.line(f"step {k} lower"))
    assert rep.ok
    grads = [("alpha", n, ga[n], rec["grad_alpha"][n], ga64[n]) for n in names]
    grads += [("beta", n, gb[n], rec["grad_beta"][n], gb64[n]) for n in beta_names]
    g_hip, bad = {}, {}
    for kind, n, got, r32, r64 in grads:
        g_hip[(kind, n)], bad[(kind, n)] = _grad_report(got, r32, r64, f"step {k} dL/d{kind}[{n}]")
    doms = sorted(set(torch.cat([m.any(dim=1).nonzero().flatten() for m in bad.values()]).tolist()))
    if doms:
        # gradients jump at kinks of the bound (a coefficient within rounding of zero decided the
        # other way): allowances from the oracle, on the domains that need them (domains are independent)
        allow = _tie_allowance(w, rec, splits, doms, bool(beta_names))
        for kind, n, got, r32, r64 in grads:
            full = torch.zeros(bad[(kind, n)].shape, dtype=torch.float64)
            full[doms] = allow[kind][n].reshape(len(doms), -1)
            _g, still = _grad_report(got, r32, r64, f"step {k} dL/d{kind}[{n}] with ties", full)
            assert not bool(still.any()), f"step {k} dL/d{kind}[{n}]: unexplained at {still.nonzero()[:8].tolist()}"
    keys = [("alpha", n) for n in names] + [("beta", n) for n in beta_names]
    for i, key in enumerate(keys):
        kind, n = key
        cur = rec[kind][n]
        g = g_hip[key].float().reshape(cur.shape)
        lo, hi = (0.0, 1.0) if kind == "alpha" else (0.0, None)
        exp = _adam_ref(cur, g, rec["exp_avg"][key], rec["exp_avg_sq"][key], int(rec["adam_step"]), lr, lo, hi)
        got = new_params[i].cpu().reshape(cur.shape)
        d = (got - exp).abs()
        bad = d > ATOL + RTOL * exp.abs()
        assert not bool(bad.any()), f"step {k} Adam update of {kind}[{n}]: {int(bad.sum())} elements, max {d.max()}"
        # against the oracle's own update: differences only where the gradient's sign is unresolved
        ref_next = rec[f"{kind}_next"][n]
        dd = (got - ref_next).abs()
        out = dd > ATOL + RTOL * ref_next.abs()
        g64 = (ga64 if kind == "alpha" else gb64)[n].double().reshape(cur.shape)
        g32 = rec[f"grad_{kind}"][n].double().reshape(cur.shape)
        # the exact update over every gradient within both fp32 gradients' error of the exact one
        delta = torch.maximum((g.double() - g64).abs(), (g32 - g64).abs())
        lo_r, hi_r = _adam_range(cur.double(), g64, delta, rec["exp_avg"][key].double(),
                                 rec["exp_avg_sq"][key].double(), int(rec["adam_step"]), lr, lo, hi)
        tol = ATOL + RTOL * ref_next.double().abs()
        inside = (got.double() >= lo_r - tol) & (got.double() <= hi_r + tol)
        announce(f"step {k} {kind}_next[{n}]: outside contract vs the oracle {int(out.sum())}/{out.numel()}, "
                 f"not reachable from the gradient's fp32 uncertainty {int((out & ~inside).sum())}")
        assert bool((~out | inside).all()), f"step {k} {kind}_next[{n}]"


def test_alpha_crown_c4_per_step():
    dev = device()
    announce("teacher-forced alpha-CROWN C4, B=32, steps 0 1 10 19 and final 20")
    w = wl.make_c4()
    _e, pre = cr.forward_ibp_trace(w.module, w.spec)
    init = ab.adaptive_alpha_init(pre)
    rec = _trajectory(w, steps=20, lr=0.1, splits=None, init=init)
    wd = wl.to_device(w, dev)
    names = list(pre.keys())
    for k in (0, 1, 10, 19, 20):
        _check_step(w, wd, rec[k], k, 0.1, None, names, [])


def test_alpha_beta_c5_per_step():
    dev = device()
    announce("teacher-forced alpha-beta-CROWN C5 domain batch, 512 domains, steps 0 1 9 and final 10")
    w = wl.subset(wl.make_c5(), 512)
    feas = ab.domain_feasible(w.module, w.spec, w.extra["splits"])
    idx = feas.nonzero().flatten()
    w = wl.Workload("C5", w.module, wl.InputSpec(value_name="input", center=w.spec.center[idx],
                                                 perturbation=w.spec.perturbation),
                    w.C[idx], w.labels[idx], {"splits": {k: v[idx] for k, v in w.extra["splits"].items()}})
    splits = w.extra["splits"]
    rec = _trajectory(w, steps=10, lr=0.2, splits=splits, init=None)
    wd = wl.to_device(w, dev)
    names = list(rec[0]["alpha"].keys())
    beta_names = [n for n in names if rec[0]["grad_beta"][n] is not None]
    for k in (0, 1, 9, 10):
        _check_step(w, wd, rec[k], k, 0.2, splits, names, beta_names)
