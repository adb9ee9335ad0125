"""Pin the CPU oracle against closed forms, known answers and brute force.

These checks are independent of the reference-generated fixtures: each one is
chosen so that a plausible slip (a swapped sign selection, a dropped bias
term, a transposed weight, a wrong relaxation intercept) fails it.
"""

import itertools

import torch

from boundflow_amd.ir import BFTaskModule, BoundTask, TaskKind, TaskOp
from boundflow_amd.spec import InputSpec, IntervalState
from oracle import alpha_beta_ref as ab
from oracle import crown_ref as cr


def _mlp(w1, b1, w2, b2):
    task = BoundTask(task_id="t0", kind=TaskKind.INTERVAL_IBP, ops=[
        TaskOp("linear", "linear1", ["input", "W1", "b1"], ["h1"]),
        TaskOp("relu", "relu1", ["h1"], ["r1"]),
        TaskOp("linear", "linear2", ["r1", "W2", "b2"], ["out"]),
    ], input_values=["input"], output_values=["out"])
    return BFTaskModule(tasks=[task], entry_task_id="t0", bindings={"params": {"W1": w1, "b1": b1, "W2": w2, "b2": b2}})


def _flat_case():
    """The explicit pre-bound fixture of tests/test_phase7a_pr10_relu_dense_reference.py:24-41."""
    pre = IntervalState(
        lower=torch.tensor([[0.2, -2.0, -1.0, -0.5], [0.1, -1.5, -0.8, -0.2]], dtype=torch.float64),
        upper=torch.tensor([[1.0, -0.1, 2.0, 0.5], [0.9, -0.2, 1.2, 0.7]], dtype=torch.float64),
    )
    torch.manual_seed(3)
    A_u = torch.randn(2, 3, 4, dtype=torch.float64)
    A_l = torch.randn(2, 3, 4, dtype=torch.float64)
    b_u = torch.randn(2, 3, dtype=torch.float64)
    b_l = torch.randn(2, 3, dtype=torch.float64)
    return pre, A_u, A_l, b_u, b_l


def test_relu_relax_closed_form():
    l = torch.tensor([0.5, -2.0, -1.0, -3.0, 0.0, -1.0])
    u = torch.tensor([2.0, -0.5, 3.0, 1.0, 0.0, 0.0])
    au, bu, al, bl = cr.relu_relax(l, u)
    # stable active, stable inactive, ambiguous chord u/(u-l) with intercept -l*u/(u-l);
    # l == u == 0 is both "active" and "inactive": the inactive assignment comes last and wins
    assert torch.equal(au, torch.tensor([1.0, 0.0, 0.75, 0.25, 0.0, 0.0]))
    assert torch.allclose(bu, torch.tensor([0.0, 0.0, 0.75, 0.75, 0.0, 0.0]))
    assert torch.equal(al, torch.tensor([1.0, 0.0, 0.0, 0.0, 0.0, 0.0]))
    assert torch.equal(bl, torch.zeros(6))


def test_alpha_gradient_matches_sign_selection_formula():
    """tests/test_phase7a_pr10_relu_dense_reference.py:132-161."""
    pre, A_u, A_l, b_u, b_l = _flat_case()
    alpha = torch.tensor([0.2, 0.3, 0.6, 0.8], dtype=torch.float64, requires_grad=True)
    out = cr.relu_backward_dense(A_u, A_l, b_u, b_l, pre=pre, name="h1", relu_alpha={"h1": alpha})
    (out[0].sum() + out[1].sum() + out[2].sum() + out[3].sum()).backward()
    amb = (pre.lower < 0) & (pre.upper > 0)
    expected = (torch.where((A_u < 0) & amb.unsqueeze(1), A_u, torch.zeros_like(A_u))
                + torch.where((A_l >= 0) & amb.unsqueeze(1), A_l, torch.zeros_like(A_l))).sum(dim=(0, 1))
    assert torch.allclose(alpha.grad, expected, atol=1e-12, rtol=1e-12)
    assert torch.equal(alpha.grad[:2], torch.zeros(2, dtype=torch.float64))


def test_dense_relu_backward_equals_fused_region_reference():
    """Dense ReLU step followed by a linear step equals the fused-region equations."""
    pre, A_u, A_l, b_u, b_l = _flat_case()
    W = torch.randn(4, 5, dtype=torch.float64)
    bias = torch.randn(4, dtype=torch.float64)
    dA_u, dA_l, nb_u, nb_l = cr.relu_backward_dense(A_u, A_l, b_u, b_l, pre=pre, name="h")
    au, bu, al, bl = cr.relu_relax(pre.lower, pre.upper)
    pu, pl, du, dl = cr.fused_relu_affine_reference(A_u, A_l, au, al, bu, bl, W, bias)
    assert torch.allclose(dA_u @ W, pu, atol=1e-12)
    assert torch.allclose(dA_l @ W, pl, atol=1e-12)
    assert torch.allclose(nb_u - b_u + (dA_u * bias).sum(2), du, atol=1e-12)
    assert torch.allclose(nb_l - b_l + (dA_l * bias).sum(2), dl, atol=1e-12)


def test_crown_bruteforce_grid_toy():
    """tests/test_phase6b_crown_ibp_mlp.py:153-175 (fp64, 41x41 grid)."""
    dt = torch.float64
    eps = 0.3
    x0 = torch.tensor([[0.2, -0.1]], dtype=dt)
    w1 = torch.tensor([[1.3, -0.7], [-0.4, 0.9]], dtype=dt)
    b1 = torch.tensor([0.05, -0.02], dtype=dt)
    w2 = torch.tensor([[-1.2, 0.8], [0.6, -0.5]], dtype=dt)
    b2 = torch.tensor([0.1, -0.3], dtype=dt)
    m = _mlp(w1, b1, w2, b2)
    crown = cr.run_crown_ibp(m, InputSpec.linf(value_name="input", center=x0, eps=eps))
    grid = torch.linspace(-eps, eps, 41, dtype=dt)
    xs = torch.stack([x0[0] + torch.stack([dx, dy]) for dx in grid for dy in grid])
    ys = torch.relu(xs @ w1.t() + b1) @ w2.t() + b2
    assert (ys >= crown.lower - 1e-9).all() and (ys <= crown.upper + 1e-9).all()
    # CROWN upper is never looser than IBP upper on this net
    env, _ = cr.forward_ibp_trace(m, InputSpec.linf(value_name="input", center=x0, eps=eps))
    assert (crown.upper <= env["out"].upper + 1e-12).all()
    # the bound is attained within grid resolution for at least one output side
    gap = torch.minimum(ys.min(0).values - crown.lower[0], crown.upper[0] - ys.max(0).values)
    assert float(gap.min()) < 0.5


def test_one_d_relu_known_answers():
    """tests/test_phase6d_alpha_crown_mlp.py:42-70 and test_phase6f (alpha-only cannot
    reach the optimum from a bad start in 0 steps, alpha-CROWN reaches lower ~ 0)."""
    one = torch.tensor([[1.0]])
    m = _mlp(one, torch.zeros(1), one, torch.zeros(1))
    spec = InputSpec.linf(value_name="input", center=torch.tensor([[0.0]]), eps=1.0)
    b0, _ = ab.run_alpha_crown(m, spec, steps=0, lr=0.2, alpha_init=0.5)
    b1, alpha = ab.run_alpha_crown(m, spec, steps=30, lr=0.2, alpha_init=0.5)
    assert abs(float(b0.upper) - 1.0) < 1e-6          # chord through (-1,0) and (1,1) at x=1
    assert abs(float(b0.lower) - (-0.5)) < 1e-6       # y >= 0.5 x at x=-1
    assert float(b1.lower) >= -1e-4 and float(b1.lower) <= 1e-6
    a = next(iter(alpha.values()))
    assert 0.0 <= float(a.min()) and float(a.max()) <= 1.0


def test_box_concretize_equals_vertex_enumeration():
    """tests/test_phase7a_pr14b_box_perturbation.py:50-72: box concretization is exact for affine maps."""
    g = torch.Generator().manual_seed(1)
    lo = torch.rand(1, 4, generator=g, dtype=torch.float64)
    hi = lo + torch.rand(1, 4, generator=g, dtype=torch.float64)
    A = torch.randn(1, 3, 4, generator=g, dtype=torch.float64)
    b = torch.randn(1, 3, generator=g, dtype=torch.float64)
    spec = InputSpec.box(value_name="input", lower=lo, upper=hi)
    lb, ub = cr.concretize_affine(spec, spec.center, cr.DenseOp(A, (4,)), b)
    verts = torch.tensor(list(itertools.product([0, 1], repeat=4)), dtype=torch.float64)
    pts = lo + verts * (hi - lo)
    vals = torch.einsum("ski,ni->nsk", A, pts) + b
    assert torch.allclose(lb, vals.min(0).values, atol=1e-12)
    assert torch.allclose(ub, vals.max(0).values, atol=1e-12)


def test_center_radius_equals_wpos_wneg_form():
    """The input-layer c/r form and the hidden-layer W+/W- form are the same interval map."""
    g = torch.Generator().manual_seed(2)
    W = torch.randn(7, 5, generator=g, dtype=torch.float64)
    b = torch.randn(7, generator=g, dtype=torch.float64)
    l = torch.randn(3, 5, generator=g, dtype=torch.float64)
    u = l + torch.rand(3, 5, generator=g, dtype=torch.float64)
    yl, yu = cr.interval_affine(l, u, W, b, {"op": "linear"})
    spec = InputSpec.box(value_name="input", lower=l, upper=u)
    cl, cu = cr.concretize_matmul(spec, spec.center, W, b)
    assert torch.allclose(yl, cl, atol=1e-12) and torch.allclose(yu, cu, atol=1e-12)


def test_branch_choice_tie_breaking():
    """alpha_beta_crown.py:145-182: first index wins within a layer, earlier layer wins ties."""
    pre = {
        "a": IntervalState(torch.tensor([[-1.0, -1.0, 0.5], [1.0, 2.0, 3.0]]), torch.tensor([[1.0, 1.0, 2.0], [2.0, 3.0, 4.0]])),
        "b": IntervalState(torch.tensor([[-1.0, -0.5], [-3.0, -1.0]]), torch.tensor([[1.0, 0.5], [0.1, 1.0]])),
    }
    assert ab.branch_choices(pre) == [("a", 0), ("b", 0)]


def test_split_application_and_infeasibility():
    pre = IntervalState(torch.tensor([[-1.0, -2.0, -0.5]]), torch.tensor([[1.0, -0.5, 2.0]]))
    out = cr.apply_relu_split(pre, torch.tensor([[1, 0, -1]], dtype=torch.int8), name="h")
    assert torch.equal(out.lower, torch.tensor([[0.0, -2.0, -0.5]]))
    assert torch.equal(out.upper, torch.tensor([[1.0, -0.5, 0.0]]))
    try:
        cr.apply_relu_split(pre, torch.tensor([[0, 1, 0]], dtype=torch.int8), name="h")
    except ValueError:
        pass
    else:
        raise AssertionError("active split on a stably inactive neuron must be infeasible")


def test_relu_influence_closed_form():
    """crown_ibp.py:1810-1833: the influence of the last ReLU is max over specs of |C W2| (both
    bounds carry C W2 there); every ReLU is covered once, with its input's shape."""
    g = torch.Generator().manual_seed(8)
    w1, b1 = torch.randn(6, 4, generator=g, dtype=torch.float64), torch.randn(6, generator=g, dtype=torch.float64)
    w2, b2 = torch.randn(3, 6, generator=g, dtype=torch.float64), torch.randn(3, generator=g, dtype=torch.float64)
    m = _mlp(w1, b1, w2, b2)
    x0 = torch.randn(2, 4, generator=g, dtype=torch.float64)
    spec = InputSpec.linf(value_name="input", center=x0, eps=0.3)
    C = torch.randn(2, 5, 3, generator=g, dtype=torch.float64)
    env, pre = cr.forward_ibp_trace(m, spec)
    infl = {}
    out = cr.crown_backward_from_trace(m, spec, interval_env=env, relu_pre=pre, linear_spec_C=C,
                                       relu_influence_out=infl)
    assert set(infl) == {"h1"} and tuple(infl["h1"].shape) == (2, 6)
    expect = (C @ w2).abs().amax(dim=1)
    assert torch.allclose(infl["h1"], expect, rtol=0, atol=1e-12)
    # the bounds are those of the plain backward
    ref = cr.crown_backward_from_trace(m, spec, interval_env=env, relu_pre=pre, linear_spec_C=C)
    assert torch.equal(out.lower, ref.lower) and torch.equal(out.upper, ref.upper)
