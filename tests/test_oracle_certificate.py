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


# ---------------------------------------------------------------------------
# conv first layers (alpha_beta_crown.py:345-389: a conv row is the one-hot output
# neuron pulled back through the conv)


def conv_first_layer_module(W, b):
    """input -> conv2d(W, b, stride 1, no padding) -> relu -> flatten -> identity linear."""
    Co, Ci, KH, KW = (int(d) for d in W.shape)
    task = BoundTask(task_id="t0", kind=TaskKind.INTERVAL_IBP, ops=[
        TaskOp("conv2d", "conv1", ["input", "W1", "b1"], ["h1"], {"stride": 1, "padding": 0, "dilation": 1,
                                                                   "groups": 1}),
        TaskOp("relu", "relu1", ["h1"], ["r1"]),
        TaskOp("flatten", "flatten", ["r1"], ["f1"], {"start_dim": 1, "end_dim": -1}),
        TaskOp("linear", "linear2", ["f1", "W2", "b2"], ["out"]),
    ], input_values=["input"], output_values=["out"])
    return task, Co


def _conv_module(W, b, in_shape):
    task, Co = conv_first_layer_module(W, b)
    ho = in_shape[1] - int(W.shape[2]) + 1
    wo = in_shape[2] - int(W.shape[3]) + 1
    n = Co * ho * wo
    return BFTaskModule(tasks=[task], entry_task_id="t0",
                        bindings={"params": {"W1": W, "b1": b, "W2": torch.eye(n), "b2": torch.zeros(n)}}), (Co, ho, wo)


def conv_jacobian(W, b, in_shape):
    """[n_out, I] rows and [n_out] offsets of conv2d (stride 1, no padding), by autograd in fp64."""
    x = torch.zeros((1,) + tuple(in_shape), dtype=torch.float64)
    f = lambda z: torch.nn.functional.conv2d(z, W.double(), b.double()).reshape(-1)  # noqa: E731
    J = torch.autograd.functional.jacobian(f, x).reshape(-1, x.numel())
    return J, f(x).detach()


def test_conv_halfspaces_are_the_conv_jacobian_rows():
    g = torch.Generator().manual_seed(6)
    in_shape = (2, 5, 4)
    W = torch.randn(3, 2, 3, 2, generator=g)
    b = torch.randn(3, generator=g)
    m, oshape = _conv_module(W, b, in_shape)
    n = oshape[0] * oshape[1] * oshape[2]
    spec = InputSpec.linf(value_name="input", center=torch.rand((1,) + in_shape, generator=g), eps=0.1)
    split = torch.zeros((1,) + oshape, dtype=torch.int8)
    picks = [0, 5, n - 1, 7]
    for i, p in enumerate(picks):
        split.view(-1)[p] = 1 if i % 2 == 0 else -1
    hs = ab.first_layer_split_halfspaces(m, spec, {"h1": split})
    J, off = conv_jacobian(W, b, in_shape)
    assert [h[1] for h in hs] == sorted(picks)
    for name, idx, a, c in hs:
        s = float(split.view(-1)[idx])
        assert name == "h1"
        assert torch.allclose(a.double(), s * J[idx], atol=1e-6)
        assert abs(float(c) - s * float(off[idx])) < 1e-6


def test_conv_certificate_matches_the_reference_fixture():
    """C3's first conv layer, one split neuron per node: the reference's flags, and its
    single-halfspace max_value where it closes the node (against the same maximum in
    fp64 from the conv's Jacobian row: s (r . x0 + b) + eps ||r||_1)."""
    from boundflow_amd import workloads as wl
    from tests.golden_util import load, workload_checksum
    g = load("cert_c3_conv")
    w = wl.subset(wl.make_c3(), 8)
    assert workload_checksum(w) == str(g["checksum"])
    eps = float(w.spec.perturbation.eps)
    W, b = w.module.params["W0"], w.module.params["b0"]
    for k in range(len(g["flag"])):
        e, n, s = int(g["example"][k]), int(g["neuron"][k]), int(g["sign"][k])
        split = torch.zeros(1, 16, 16, 16, dtype=torch.int8)
        split.view(-1)[n] = s
        spec = InputSpec.linf(value_name="input", center=w.spec.center[e:e + 1], eps=eps)
        got = ab.split_certificate(w.module, spec, {"h0": split})[0]
        assert int(got) == int(g["flag"][k]), k
        # the single halfspace's maximum over the ball, in fp64
        one = torch.zeros(1, 16, 16, 16, dtype=torch.float64)
        one.view(-1)[n] = 1.0
        row = torch.nn.functional.conv_transpose2d(one, W.double(), stride=2, padding=1).reshape(-1)
        ch = n // 256
        vmax = s * (float(row @ w.spec.center[e].double().reshape(-1)) + float(b[ch])) + eps * float(row.abs().sum())
        if int(g["flag"][k]):
            assert abs(float(g["max_value"][k]) - vmax) <= 1e-5 * abs(vmax) + 1e-5, (k, float(g["max_value"][k]), vmax)
        assert (vmax < -1e-6) == bool(g["flag"][k])


def _conv_lp_trials(seed, trials):
    """Random conv first layers on a 1x3x3 input in the box [-1, 1]^9 with 2-4 split
    neurons each (each halfspace feasible alone: the IBP trace passes)."""
    g = torch.Generator().manual_seed(seed)
    in_shape = (1, 3, 3)
    for trial in range(trials):
        W = torch.randn(3, 1, 2, 2, generator=g)
        b = torch.randn(3, generator=g) * 0.6 - 0.9
        m, oshape = _conv_module(W, b, in_shape)
        n = oshape[0] * oshape[1] * oshape[2]
        k = int(torch.randint(2, 5, (1,), generator=g))
        split = torch.zeros(1, n, dtype=torch.int8)
        split[0, torch.randperm(n, generator=g)[:k]] = 1
        spec = InputSpec.linf(value_name="input", center=torch.zeros((1,) + in_shape), eps=1.0)
        sp = {"h1": split.reshape((1,) + oshape)}
        try:
            cr.forward_ibp_trace(m, spec, relu_split_state=sp)
        except ValueError:
            continue
        yield trial, W, b, m, spec, sp, split


def test_conv_certificate_verdicts_are_sound_against_an_lp():
    """Two or more split neurons on a conv first layer (where the reference's stacking of
    conv rows cannot broadcast): every set the oracle closes has no point in the box
    (exact LP on the conv's Jacobian rows), and the verdicts equal those of the same
    halfspaces written as a linear first layer (the path the reference's known answers pin)."""
    found = 0
    for trial, W, b, m, spec, sp, split in _conv_lp_trials(31, 80):
        got = ab.split_certificate(m, spec, sp)[0]
        J, off = conv_jacobian(W, b, (1, 3, 3))
        rows = split[0].nonzero().flatten()
        lin = first_layer_module(J.float(), off.float())
        lin_spec = InputSpec.linf(value_name="input", center=torch.zeros(1, 9), eps=1.0)
        assert got == ab.split_certificate(lin, lin_spec, {"h1": split})[0], trial
        if got:
            found += 1
            feas = _lp_feasible(J[rows].numpy(), off[rows].numpy(), [-1.0] * 9, [1.0] * 9)
            assert not feas, f"trial {trial}: certificate on a feasible conv halfspace set"
    assert found >= 3, found
