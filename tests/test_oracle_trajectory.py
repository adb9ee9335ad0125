"""The trajectory checks of oracle/trajectory.py on the CPU: an exact trajectory
passes them, and each planted mistake (in the oracle's own recorded trajectory,
standing in for a device record) is caught.  The Adam enclosure is checked
against torch's Adam: exact with zero radii, and containing every sampled
history inside the radii."""

import copy

import pytest
import torch

from boundflow_amd import workloads as wl
from oracle import alpha_beta_ref as ab
from oracle import trajectory as tt

LR = 0.2
STEPS = 3


@pytest.fixture(scope="module")
def case():
    w = wl.subset(wl.make_c5(eps=0.004, depth=2, label_mode="predicted"), 6)
    assert bool(ab.domain_feasible(w.module, w.spec, w.extra["splits"]).all())
    rec = []
    best = ab.run_alpha_beta_crown(w.module, w.spec, linear_spec_C=w.C, relu_split_state=w.extra["splits"],
                                   steps=STEPS, lr=LR, per_batch_params=True, record=rec)[0]
    names = list(rec[0]["alpha"].keys())
    beta_names = [n for n in names if rec[0]["grad_beta"][n] is not None]
    return w, rec, best.lower, names, beta_names


def _quiet(_msg):
    pass


def test_exact_trajectory_passes(case):
    w, rec, final, names, beta_names = case
    sh = tt.shadow_check(w, rec, LR, names, beta_names, "exact", final_lower=final, log=_quiet)
    out = tt.divergence_trace(w, rec, rec, sh, LR, names, beta_names, list(range(w.batch)), "exact", log=_quiet)
    assert all(k == -1 for k, _n, _c in out.values())


def test_planted_gradient_error_is_caught(case):
    w, rec, final, names, beta_names = case
    bad = copy.deepcopy(rec)
    g = bad[1]["grad_alpha"][names[0]]
    g.view(-1)[17] += 1e-3 * float(g.abs().max())
    with pytest.raises(AssertionError, match="outside their fp32 uncertainty"):
        tt.shadow_check(w, bad, LR, names, beta_names, "planted gradient", log=_quiet)


def test_planted_beta_gradient_error_is_caught(case):
    w, rec, final, names, beta_names = case
    bad = copy.deepcopy(rec)
    n = beta_names[0]
    g = bad[0]["grad_beta"][n]
    j = int(g.reshape(-1).abs().argmax())
    g.view(-1)[j] *= 1.001
    with pytest.raises(AssertionError, match="outside their fp32 uncertainty"):
        tt.shadow_check(w, bad, LR, names, beta_names, "planted beta gradient", log=_quiet)


def test_planted_bound_error_is_caught(case):
    w, rec, final, names, beta_names = case
    bad = copy.deepcopy(rec)
    bad[2]["lower"][3, 4] += 1e-4 * (1.0 + float(bad[2]["lower"][3, 4].abs()))
    with pytest.raises(AssertionError, match="lower bounds at HIP states"):
        tt.shadow_check(w, bad, LR, names, beta_names, "planted bound", log=_quiet)


def test_planted_adam_error_is_caught(case):
    w, rec, final, names, beta_names = case
    bad = copy.deepcopy(rec)
    bad[1]["alpha_next"][names[1]].view(-1)[5] += 1e-4
    with pytest.raises(AssertionError, match="Adam update"):
        tt.shadow_check(w, bad, LR, names, beta_names, "planted Adam", log=_quiet)


def test_planted_best_of_error_is_caught(case):
    w, rec, final, names, beta_names = case
    metrics = torch.stack([r["lower"].mean(dim=1) for r in rec])
    worst = metrics.argmin(dim=0)
    wrong = torch.stack([rec[int(worst[d])]["lower"][d] for d in range(w.batch)])
    with pytest.raises(AssertionError, match="best-of"):
        tt.shadow_check(w, rec, LR, names, beta_names, "planted best-of", final_lower=wrong, log=_quiet)


def test_planted_divergence_is_caught(case):
    w, rec, final, names, beta_names = case
    sh = tt.shadow_check(w, rec, LR, names, beta_names, "exact", log=_quiet)
    bad = copy.deepcopy(rec)
    a = bad[1]["alpha_next"][names[0]]
    j = int(rec[1]["grad_alpha"][names[0]][2].abs().argmax())
    a[2, j] = 1.0 - a[2, j]    # a far jump of a parameter with a large, well-resolved gradient
    with pytest.raises(AssertionError, match="Adam-reachable"):
        tt.divergence_trace(w, bad, rec, sh, LR, names, beta_names, [2], "planted divergence", log=_quiet)


def test_adam_enclosure_matches_torch_and_contains_samples():
    g = torch.Generator().manual_seed(3)
    n, t = 257, 5
    p = torch.rand(n, generator=g, dtype=torch.float64)
    hist = [torch.randn(n, generator=g, dtype=torch.float64) * torch.logspace(-6, 1, n, dtype=torch.float64)
            for _ in range(t)]
    zero = [torch.zeros(n, dtype=torch.float64)] * t
    lo, hi = tt.adam_reach(p, hist, zero, 0.1, 0.0, 1.0)
    # torch Adam over the same history, ending with the step from p
    q = torch.zeros(n, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.Adam([q], lr=0.1)
    for j, gj in enumerate(hist):
        if j == t - 1:
            with torch.no_grad():
                q.copy_(p)
        q.grad = gj.clone()
        opt.step()
    exp = q.detach().clamp(0.0, 1.0)
    assert torch.allclose(lo, exp, rtol=0, atol=1e-12) and torch.allclose(hi, exp, rtol=0, atol=1e-12)
    radii = [h.abs() * 0.5 + 1e-7 for h in hist]
    lo, hi = tt.adam_reach(p, hist, radii, 0.1, 0.0, 1.0)
    for _ in range(64):
        qq = torch.zeros(n, dtype=torch.float64, requires_grad=True)
        opt = torch.optim.Adam([qq], lr=0.1)
        for j, (c, r) in enumerate(zip(hist, radii)):
            if j == t - 1:
                with torch.no_grad():
                    qq.copy_(p)
            qq.grad = c + (2.0 * torch.rand(n, generator=g, dtype=torch.float64) - 1.0) * r
            opt.step()
        v = qq.detach().clamp(0.0, 1.0)
        assert bool(((v >= lo - 1e-12) & (v <= hi + 1e-12)).all())
