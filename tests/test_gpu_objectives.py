"""Objectives ("upper", "gap", "both", "lower") and spec reductions ("mean",
"min", "softmin") of the HIP alpha-beta loop against the reference's
run_alpha_beta_crown_mlp (fixture objectives_mlp, 8 Adam steps, per-domain and
shared parameters).  Whole 8-step trajectories: the counts at the contract are
reported and every bound must be within 1e-4 of the reference or fp64-explained
there (the fp64 oracle run with the same options), with identical verdicts.
The one-step runs (the initial evaluation and one Adam step) are held to the
contract, fp64-explained."""

import pytest
import torch

from boundflow_amd import alpha_beta as hab
from boundflow_amd import workloads as wl
from oracle import alpha_beta_ref as ab
from oracle import parity
from tests.golden_util import ALPHA_CROWN_OBJECTIVE_CASES, OBJECTIVE_CASES, load, objective_workload, t
from tests.gpu_util import announce, device

pytestmark = pytest.mark.gpu


def _run_hip(w, splits, dev, steps, kw):
    wd = wl.to_device(w, dev)
    b, _a, _bt, _st = hab.run_alpha_beta_crown_mlp(wd.module, wd.spec, linear_spec_C=wd.C,
                                                   relu_split_state={k: v.to(dev) for k, v in splits.items()},
                                                   steps=steps, lr=0.1, **kw)
    torch.cuda.synchronize()
    return b.lower.cpu(), b.upper.cpu()


def _run_oracle(w, splits, steps, kw):
    b, _a, _bt, _ch = ab.run_alpha_beta_crown(w.module, w.spec, linear_spec_C=w.C, relu_split_state=splits,
                                              steps=steps, lr=0.1, **kw)
    return b.lower.detach(), b.upper.detach()


@pytest.mark.parametrize("case", list(OBJECTIVE_CASES))
def test_objective_trajectory_matches_reference(case):
    dev = device()
    announce(f"alpha-beta objective {case}, 8 steps")
    g = load("objectives_mlp")
    w, splits = objective_workload()
    kw = OBJECTIVE_CASES[case]
    lo, hi = _run_hip(w, splits, dev, 8, kw)
    ref_lo, ref_hi = t(g[f"{case}_lower"]), t(g[f"{case}_upper"])
    w64 = parity.to_float64(w)
    e_lo, e_hi = _run_oracle(w64, splits, 8, kw)
    for what, got, ref, e in (("lower", lo, ref_lo, e_lo), ("upper", hi, ref_hi, e_hi)):
        strict = parity.compare(got, ref, None)
        rep = parity.compare(got, ref, e, rtol=1e-4, atol=1e-4)
        announce(f"  {case} {what}: at the contract {strict.strict_violations}/{strict.n} outside; "
                 + rep.line("at 1e-4"))
        assert rep.ok
    mism, _flips, ties = parity.verdict_parity(lo, ref_lo, e_lo)
    assert mism == 0


@pytest.mark.parametrize("case", list(OBJECTIVE_CASES))
def test_objective_one_step_at_the_contract(case):
    dev = device()
    announce(f"alpha-beta objective {case}, 1 step, contract")
    w, splits = objective_workload()
    kw = OBJECTIVE_CASES[case]
    lo, hi = _run_hip(w, splits, dev, 1, kw)
    r_lo, r_hi = _run_oracle(w, splits, 1, kw)
    e_lo, e_hi = _run_oracle(parity.to_float64(w), splits, 1, kw)
    for what, got, ref, e in (("lower", lo, r_lo, e_lo), ("upper", hi, r_hi, e_hi)):
        rep = parity.compare(got, ref, e)
        announce(f"  {case} {what}: " + rep.line("1 step"))
        assert rep.ok


@pytest.mark.parametrize("case", list(ALPHA_CROWN_OBJECTIVE_CASES))
def test_alpha_crown_objective_matches_reference(case):
    """HIP run_alpha_crown_mlp (shared alpha) with each objective against the
    reference's run_alpha_crown_mlp (fixture alpha_crown_objectives), 8 Adam steps:
    bounds within 1e-4 of the reference or fp64-explained there, contract counts
    reported, identical verdicts."""
    dev = device()
    announce(f"alpha-crown objective {case}, 8 steps")
    g = load("alpha_crown_objectives")
    w, splits = objective_workload()
    kw = ALPHA_CROWN_OBJECTIVE_CASES[case]
    wd = wl.to_device(w, dev)
    b, _alpha, _st = hab.run_alpha_crown_mlp(wd.module, wd.spec, linear_spec_C=wd.C,
                                             relu_split_state={k: v.to(dev) for k, v in splits.items()},
                                             steps=8, lr=0.1, **kw)
    torch.cuda.synchronize()
    lo, hi = b.lower.cpu(), b.upper.cpu()
    w64 = parity.to_float64(w)
    e, _ea = ab.run_alpha_crown(w64.module, w64.spec, linear_spec_C=w64.C, relu_split_state=splits, steps=8, lr=0.1,
                                **kw)
    for what, got, ref, ex in (("lower", lo, t(g[f"{case}_lower"]), e.lower.detach()),
                               ("upper", hi, t(g[f"{case}_upper"]), e.upper.detach())):
        strict = parity.compare(got, ref, None)
        rep = parity.compare(got, ref, ex, rtol=1e-4, atol=1e-4)
        announce(f"  {case} {what}: at the contract {strict.strict_violations}/{strict.n} outside; "
                 + rep.line("at 1e-4"))
        assert rep.ok
    mism, _flips, _ties = parity.verdict_parity(lo, t(g[f"{case}_lower"]), e.lower.detach())
    assert mism == 0
