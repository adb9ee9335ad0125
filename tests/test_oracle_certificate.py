"""Pin the oracle's first-layer split certificate (oracle/alpha_beta_ref.py
``split_certificate``, restating alpha_beta_crown.py:391-532):

* the reference's own known answers (tests/test_phase6f_alpha_beta_crown_pr1.py:53-93):
  two opposite halfspaces on [-1, 1]^2 and a non-pairwise triple are infeasible,
  though each halfspace alone is feasible (so the IBP trace does not raise);
* a feasible set of the same shapes is never declared infeasible;
* one halfspace: infeasible exactly when its maximum over the box (by vertex
  enumeration) is below -tol;
* soundness against an exact linear program (scipy's HiGHS): every set the
  certificate declares infeasible has no point in the input box.
The whole-search fixtures with certificate closures (bab_solve_cert_*) pin it
inside the BaB loop (tests/test_oracle_bab.py)."""

import itertools

import numpy as np
import pytest
import torch

from boundflow_amd.ir import BFTaskModule, BoundTask, TaskKind, TaskOp
from boundflow_amd.spec import InputSpec
from oracle import alpha_beta_ref as ab
from oracle import crown_ref as cr


def first_layer_module(w, b):
    """input -> linear -> relu -> identity linear (the reference tests' module)."""
    h = int(w.shape[0])
    task = BoundTask(task_id="t0", kind=TaskKind.INTERVAL_IBP, ops=[
        TaskOp("linear", "linear1", ["input", "W1", "b1"], ["h1"]),
        TaskOp("relu", "relu1", ["h1"], ["r1"]),
        TaskOp("linear", "linear2", ["r1", "W2", "b2"], ["out"]),
    ], input_values=["input"], output_values=["out"])
    return BFTaskModule(tasks=[task], entry_task_id="t0",
                        bindings={"params": {"W1": w, "b1": b, "W2": torch.eye(h), "b2": torch.zeros(h)}})


KATS = {
    # name: (W, b, split, infeasible)
    "opposite_pair": ([[1.0, 1.0], [-1.0, -1.0]], [-1.2, -1.2], [1, 1], True),
    "non_pairwise_triple": ([[1.0, 0.0], [0.0, 1.0], [-1.0, -1.0]], [-0.6, -0.6, -0.6], [1, 1, 1], True),
    "feasible_pair": ([[1.0, 0.0], [0.0, 1.0]], [-0.6, -0.6], [1, 1], False),
    "feasible_mixed_signs": ([[1.0, 1.0], [-1.0, -1.0]], [-1.2, -1.2], [1, -1], False),
}


@pytest.mark.parametrize("name", list(KATS))
def test_known_answers(name):
    W, b, s, expect = KATS[name]
    m = first_layer_module(torch.tensor(W), torch.tensor(b))
    spec = InputSpec.linf(value_name="input", center=torch.zeros(1, 2), eps=1.0)
    split = {"h1": torch.tensor([s], dtype=torch.int8)}
    got, _why = ab.split_certificate(m, spec, split)
    assert got == expect
    # the IBP trace alone does not see it: every halfspace is feasible by itself
    cr.forward_ibp_trace(m, spec, relu_split_state=split)
    # the alpha-beta entry point returns the reference's infeasible result
    out = ab.run_alpha_beta_crown(m, spec, linear_spec_C=None, relu_split_state=split, steps=0,
                                  return_feasibility=True)
    assert out[4] == ("infeasible" if expect else "unknown")
    if expect:
        assert tuple(out[0].lower.shape) == (1, 1) and float(out[0].lower.abs().max()) == 0.0


def test_box_input_known_answer():
    W, b, s, _ = KATS["opposite_pair"]
    m = first_layer_module(torch.tensor(W), torch.tensor(b))
    spec = InputSpec.box(value_name="input", lower=torch.full((1, 2), -1.0), upper=torch.full((1, 2), 1.0))
    assert ab.split_certificate(m, spec, {"h1": torch.tensor([s], dtype=torch.int8)})[0]
    # a smaller box where x1 + x2 >= 1.2 is impossible even alone: one halfspace suffices
    spec2 = InputSpec.box(value_name="input", lower=torch.full((1, 2), -1.0), upper=torch.full((1, 2), 0.5))
    assert ab.split_certificate(m, spec2, {"h1": torch.tensor([[1, 0]], dtype=torch.int8)})[0]


def test_single_halfspace_matches_vertex_enumeration():
    g = torch.Generator().manual_seed(3)
    for trial in range(40):
        d = 3
        w = torch.randn(1, d, generator=g)
        b = torch.randn(1, generator=g) * 2
        x0 = torch.rand(1, d, generator=g)
        eps = 0.3
        s = 1 if trial % 2 == 0 else -1
        m = first_layer_module(w, b)
        spec = InputSpec.linf(value_name="input", center=x0, eps=eps)
        got = ab.split_certificate(m, spec, {"h1": torch.tensor([[s]], dtype=torch.int8)})[0]
        verts = torch.tensor(list(itertools.product([-1.0, 1.0], repeat=d)), dtype=torch.float64)
        xs = x0.double() + eps * verts
        vmax = float((s * (xs @ w.double().t() + b.double())).max())
        if abs(vmax + 1e-6) > 1e-5:   # away from the tolerance boundary
            assert got == (vmax < -1e-6), (trial, vmax)


def _lp_feasible(a, c, lo, hi) -> bool:
    """Exact: is there x in [lo, hi] with a x + c >= 0 for every row?"""
    from scipy.optimize import linprog
    res = linprog(np.zeros(a.shape[1]), A_ub=-a, b_ub=c, bounds=list(zip(lo, hi)), method="highs")
    return res.status == 0


def test_infeasible_verdicts_are_sound_against_an_lp():
    g = torch.Generator().manual_seed(11)
    found = 0
    for trial in range(60):
        d, k = 2, int(torch.randint(2, 5, (1,), generator=g))
        w = torch.randn(k, d, generator=g)
        b = torch.randn(k, generator=g) * 0.5 - 0.4
        x0 = torch.zeros(1, d)
        spec = InputSpec.linf(value_name="input", center=x0, eps=1.0)
        s = torch.ones(1, k, dtype=torch.int8)
        m = first_layer_module(w, b)
        try:
            cr.forward_ibp_trace(m, spec, relu_split_state={"h1": s})
        except ValueError:
            continue   # IBP alone closes it; the certificate is not what decides
        got = ab.split_certificate(m, spec, {"h1": s})[0]
        feas = _lp_feasible(w.double().numpy(), b.double().numpy(), [-1.0] * d, [1.0] * d)
        if got:
            found += 1
            assert not feas, f"trial {trial}: certificate on a feasible set"
    assert found >= 1


# Known answers over L2 and L1 balls of radius 1 at the origin, fixed by geometry:
# x1 >= 0.6 and x2 >= 0.6 meet inside the Linf and L2 balls ((0.6, 0.6) has L2 norm
# 0.85) but not inside the L1 ball (|x1| + |x2| >= 1.2); at 0.75 they miss the L2 ball
# too (0.75 * sqrt(2) > 1).  Three unit normals at 0/120/240 degrees sum to zero, so
# a_i . x >= 0.49 for all three has no point in any set (the reference's L2 case,
# tests/test_phase6f_alpha_beta_crown_pr1.py:96-118); at -0.1 the origin satisfies all.
_DIRS = [[1.0, 0.0], [-0.5, 0.8660254], [-0.5, -0.8660254]]
LP_KATS = {
    # name: (W, b, split, {p: infeasible})
    "pair_0.6": ([[1.0, 0.0], [0.0, 1.0]], [-0.6, -0.6], [1, 1], {"inf": False, 2: False, 1: True}),
    "pair_0.75": ([[1.0, 0.0], [0.0, 1.0]], [-0.75, -0.75], [1, 1], {"inf": False, 2: True, 1: True}),
    "three_directions": (_DIRS, [-0.49] * 3, [1, 1, 1], {"inf": True, 2: True, 1: True}),
    "three_directions_feasible": (_DIRS, [0.1] * 3, [1, 1, 1], {"inf": False, 2: False, 1: False}),
    "single_1.2": ([[1.0, 1.0]], [-1.2], [1], {"inf": False, 2: False, 1: True}),
    "single_1.5": ([[1.0, 1.0]], [-1.5], [1], {"inf": False, 2: True, 1: True}),
}


def lp_spec(p, center, eps=1.0):
    from boundflow_amd.spec import LpBallPerturbation
    return InputSpec(value_name="input", center=center, perturbation=LpBallPerturbation(p=p, eps=eps))


@pytest.mark.parametrize("p", ["inf", 2, 1])
@pytest.mark.parametrize("name", list(LP_KATS))
def test_lp_ball_known_answers(name, p):
    W, b, s, expect = LP_KATS[name]
    m = first_layer_module(torch.tensor(W), torch.tensor(b))
    spec = lp_spec(p, torch.zeros(1, 2))
    split = {"h1": torch.tensor([s], dtype=torch.int8)}
    assert ab.split_certificate(m, spec, split)[0] == expect[p]
    out = ab.run_alpha_beta_crown(m, spec, linear_spec_C=None, relu_split_state=split, steps=0,
                                  return_feasibility=True)
    assert out[4] == ("infeasible" if expect[p] else "unknown")


@pytest.mark.parametrize("p", [2, 1])
def test_lp_ball_infeasible_verdicts_are_sound(p):
    """No point of a dense sample of the ball satisfies every halfspace of a set the
    certificate closes (the L1 ball's vertices and edges are in the sample)."""
    g = torch.Generator().manual_seed(17 + p)
    r = torch.linspace(0, 1, 81, dtype=torch.float64)
    th = torch.linspace(0, 2 * torch.pi, 721, dtype=torch.float64)[:-1]
    rr, tt = torch.meshgrid(r, th, indexing="ij")
    u = torch.stack([torch.cos(tt), torch.sin(tt)], -1).reshape(-1, 2)
    if p == 1:
        u = u / u.abs().sum(-1, keepdim=True)
    pts = rr.reshape(-1, 1) * u
    found = 0
    for trial in range(60):
        k = int(torch.randint(2, 5, (1,), generator=g))
        w = torch.randn(k, 2, generator=g)
        b = torch.randn(k, generator=g) * 0.5 - 0.4
        m = first_layer_module(w, b)
        spec = lp_spec(p, torch.zeros(1, 2))
        s = torch.ones(1, k, dtype=torch.int8)
        try:
            cr.forward_ibp_trace(m, spec, relu_split_state={"h1": s})
        except ValueError:
            continue
        if ab.split_certificate(m, spec, {"h1": s})[0]:
            found += 1
            inside = ((pts @ w.double().t() + b.double()) >= 0).all(dim=1)
            assert not bool(inside.any()), f"trial {trial}: certificate on a set with a point in the ball"
    assert found >= 1
