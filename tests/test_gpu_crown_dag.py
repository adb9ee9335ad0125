"""HIP parity tests of CROWN-IBP on DAG networks (residual add, concat, fan-out):
``run_crown_ibp_mlp`` on a task that is not a chain runs the general backward of
``boundflow_amd.crown_dag`` and must match the oracle (crown_ibp.py:1669-2051),
whose DAG pieces are pinned in tests/test_oracle_dag.py."""

import pytest
import torch

from boundflow_amd import alpha_beta as hab
from boundflow_amd import crown as hc
from boundflow_amd import crown_dag
from boundflow_amd import workloads as wl
from oracle import alpha_beta_ref as ab
from oracle import crown_ref as cr
from oracle import parity
from tests.golden_util import dag_case, load, t, workload_checksum
from tests.gpu_util import announce, assert_bounds_close, assert_parity, assert_verdicts, device
from tests.test_gpu_conv_alpha import _grad_close, _oracle_grads, _sign_tie_allowance

pytestmark = pytest.mark.gpu


def _check(w, dev, what, **kw):
    """HIP bounds of workload w against the fp32 oracle, fp64 as the cancellation referee."""
    wd = wl.to_device(w, dev)
    kw_dev = {k: ({n: t.to(dev) for n, t in v.items()} if isinstance(v, dict) else v) for k, v in kw.items()}
    got = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C, **kw_dev)
    torch.cuda.synchronize()
    ref = cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C, **kw)
    w64 = parity.to_float64(w)
    kw64 = {k: ({n: (t.double() if t.is_floating_point() else t) for n, t in v.items()} if isinstance(v, dict) else v)
            for k, v in kw.items()}
    ref64 = cr.run_crown_ibp(w64.module, w64.spec, linear_spec_C=w64.C, **kw64)
    assert_parity(got.lower, ref.lower, ref64.lower, f"{what} lower")
    assert_parity(got.upper, ref.upper, ref64.upper, f"{what} upper")
    assert_verdicts(got.lower, ref.lower, ref64.lower, what)
    return got


@pytest.mark.parametrize("kind", wl.DAG_KINDS)
@pytest.mark.parametrize("box", [False, True])
def test_dag_crown_matches_oracle(kind, box):
    dev = device()
    announce(f"DAG CROWN {kind} box={box}")
    w = wl.make_dag(kind, seed=3, batch=6, eps=0.03, box=box, blocks=2)
    _check(w, dev, f"{kind} box={box}")


@pytest.mark.parametrize("kind", wl.DAG_KINDS)
@pytest.mark.parametrize("box", [False, True])
def test_dag_crown_matches_reference_fixture(kind, box):
    """HIP DAG CROWN against the reference's run_crown_ibp_mlp on the same network
    (fixture crown_dag_<kind>[_box]), fp64-explained at the contract, same verdicts."""
    dev = device()
    tag = f"crown_dag_{kind}{'_box' if box else ''}"
    announce(f"DAG CROWN {tag} vs reference fixture")
    g = load(tag)
    w = dag_case(kind, box)
    assert workload_checksum(w) == str(g["checksum"])
    wd = wl.to_device(w, dev)
    got = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
    torch.cuda.synchronize()
    w64 = parity.to_float64(w)
    ref64 = cr.run_crown_ibp(w64.module, w64.spec, linear_spec_C=w64.C)
    assert_parity(got.lower, t(g["lower"]), ref64.lower, f"{tag} lower")
    assert_parity(got.upper, t(g["upper"]), ref64.upper, f"{tag} upper")
    assert_verdicts(got.lower, t(g["lower"]), ref64.lower, tag)


@pytest.mark.parametrize("kind", wl.DAG_KINDS)
def test_dag_ibp_trace_matches_oracle(kind):
    dev = device()
    announce(f"DAG IBP trace {kind}")
    w = wl.make_dag(kind, seed=4, batch=5, eps=0.05, blocks=2)
    wd = wl.to_device(w, dev)
    trace = hc.forward_ibp_trace(wd.module, wd.spec)
    assert isinstance(trace, crown_dag.DagTrace)
    _env, pre = cr.forward_ibp_trace(w.module, w.spec)
    assert list(trace.relu_pre.keys()) == list(pre.keys())
    for name, st in pre.items():
        assert_bounds_close(trace.relu_pre[name].lower, st.lower, f"{kind} relu_pre[{name}].lower", atol=1e-5)
        assert_bounds_close(trace.relu_pre[name].upper, st.upper, f"{kind} relu_pre[{name}].upper", atol=1e-5)


def test_dag_crown_identity_spec_and_from_trace():
    """No spec matrix (C = I over the 10 outputs), and the same bound through
    run_crown_ibp_mlp_from_forward_trace on the DAG trace."""
    dev = device()
    announce("DAG CROWN residual_mlp, C = I")
    w = wl.make_dag("residual_mlp", seed=5, batch=4, eps=0.03, blocks=3)
    wd = wl.to_device(w, dev)
    got = hc.run_crown_ibp_mlp(wd.module, wd.spec)
    trace = hc.forward_ibp_trace(wd.module, wd.spec)
    again = hc.run_crown_ibp_mlp_from_forward_trace(wd.module, wd.spec, trace=trace)
    torch.cuda.synchronize()
    ref = cr.run_crown_ibp(w.module, w.spec)
    ref64 = cr.run_crown_ibp(parity.to_float64(w).module, parity.to_float64(w).spec)
    assert_parity(got.lower, ref.lower, ref64.lower, "C=I lower")
    assert_parity(got.upper, ref.upper, ref64.upper, "C=I upper")
    assert torch.equal(got.lower, again.lower) and torch.equal(got.upper, again.upper)


@pytest.mark.parametrize("kind", ["residual_mlp", "projection_skip_cnn"])
def test_dag_crown_with_alpha_beta_and_splits(kind):
    """Lower-slope override, lower-bound split coefficient and split state on every ReLU."""
    dev = device()
    announce(f"DAG CROWN {kind} with alpha, beta coefficient and splits")
    w = wl.make_dag(kind, seed=6, batch=4, eps=0.04, blocks=2)
    _env, pre = cr.forward_ibp_trace(w.module, w.spec)
    g = torch.Generator().manual_seed(9)
    alpha, add, splits = {}, {}, {}
    for name in pre:
        # split only neurons that are ambiguous given the splits of the ReLUs before (feasible)
        _env, cur = cr.forward_ibp_trace(w.module, w.spec, relu_split_state=dict(splits))
        st = cur[name]
        shape = tuple(st.lower.shape)
        alpha[name] = torch.rand(shape, generator=g)
        add[name] = torch.randn(shape, generator=g) * 0.1
        amb = (st.lower < 0) & (st.upper > 0)
        choice = torch.randint(-1, 2, shape, generator=g).to(torch.int8)
        splits[name] = torch.where(amb, choice, torch.zeros_like(choice))
    _check(w, dev, f"{kind} alpha/beta/splits", relu_alpha=alpha, relu_pre_add_coeff_l=add,
           relu_split_state=splits)


def test_dag_crown_larger_residual_network():
    """A residual MLP at a size where the contraction runs on full MFMA tiles."""
    dev = device()
    announce("DAG CROWN residual_mlp 256 wide, 3 blocks, B=32")
    w = wl.make_dag("residual_mlp", seed=7, batch=32, eps=0.001, n_in=256, hidden=512, blocks=3)
    _check(w, dev, "residual 256x512x3")


def test_dag_crown_constant_add_operand():
    """A per-sample constant operand of add folds into the bias (crown_ibp.py:1937-1950)."""
    from boundflow_amd.ir import BFTaskModule, BoundTask, TaskKind, TaskOp
    dev = device()
    announce("DAG CROWN with a constant add operand")
    g = torch.Generator().manual_seed(12)
    B = 3
    params = {"W1": torch.randn(20, 12, generator=g) * 0.3, "b1": torch.randn(20, generator=g) * 0.1,
              "P": torch.randn(B, 20, generator=g) * 0.2, "W2": torch.randn(10, 20, generator=g) * 0.3}
    ops = [TaskOp("linear", "lin1", ["input", "W1", "b1"], ["h"]), TaskOp("add", "add0", ["h", "P"], ["s"]),
           TaskOp("relu", "relu0", ["s"], ["r"]), TaskOp("linear", "lin2", ["r", "W2"], ["out"])]
    task = BoundTask(task_id="t0", kind=TaskKind.INTERVAL_IBP, ops=ops, input_values=["input"],
                     output_values=["out"])
    module = BFTaskModule(tasks=[task], entry_task_id="t0", bindings={"params": params})
    x = torch.rand(B, 12, generator=g)
    from boundflow_amd.spec import InputSpec
    w = wl.Workload("const_add", module, InputSpec.linf(value_name="input", center=x, eps=0.05),
                    wl.margin_spec(torch.tensor([1, 4, 7])), torch.tensor([1, 4, 7]))
    _check(w, dev, "constant add")


def test_dag_crown_rejects_broadcast_add():
    from boundflow_amd.ir import BFTaskModule, BoundTask, TaskKind, TaskOp
    from boundflow_amd.spec import InputSpec
    dev = device()
    announce("DAG CROWN broadcast add -> NotImplementedError")
    params = {"W1": torch.ones(4, 3, device=dev), "c": torch.ones(4, device=dev), "W2": torch.ones(2, 4, device=dev)}
    ops = [TaskOp("linear", "lin1", ["input", "W1"], ["h1"]), TaskOp("add", "add0", ["h1", "c"], ["s"]),
           TaskOp("linear", "lin2", ["s", "W2"], ["out"])]
    task = BoundTask(task_id="t0", kind=TaskKind.INTERVAL_IBP, ops=ops, input_values=["input"],
                     output_values=["out"])
    module = BFTaskModule(tasks=[task], entry_task_id="t0", bindings={"params": params})
    spec = InputSpec.linf(value_name="input", center=torch.rand(2, 3, device=dev), eps=0.1)
    with pytest.raises(NotImplementedError, match="same-shape"):
        hc.run_crown_ibp_mlp(module, spec)


def _feasible_splits(w, g):
    """Random splits on neurons ambiguous given the splits of the ReLUs before them."""
    _env, pre = cr.forward_ibp_trace(w.module, w.spec)
    splits = {}
    for name in pre:
        _env, cur = cr.forward_ibp_trace(w.module, w.spec, relu_split_state=dict(splits))
        st = cur[name]
        amb = (st.lower < 0) & (st.upper > 0)
        choice = torch.randint(-1, 2, tuple(st.lower.shape), generator=g).to(torch.int8)
        splits[name] = torch.where(amb, choice, torch.zeros_like(choice))
    return splits


@pytest.mark.parametrize("kind,with_beta", [("residual_mlp", True), ("residual_mlp", False),
                                            ("projection_skip_cnn", True), ("feature_concat_mlp", False),
                                            ("channel_concat_cnn", True)])
def test_dag_lower_bound_gradients_match_autograd(kind, with_beta):
    """The reverse pass of the DAG backward (crown_dag.lower_grad_pass) against autograd
    through the oracle's DAG backward: dL/dalpha and dL/dbeta for L = -sum_d mean_s lb."""
    dev = device()
    announce(f"DAG alpha/beta gradient pass vs autograd: {kind} beta={with_beta}")
    g = torch.Generator().manual_seed(31)
    w = wl.make_dag(kind, seed=8, batch=3, eps=0.03, blocks=2)
    splits = _feasible_splits(w, g) if with_beta else None
    _env, pre = cr.forward_ibp_trace(w.module, w.spec, relu_split_state=splits)
    alpha = {k: torch.rand(v.lower.shape, generator=g) for k, v in pre.items()}
    beta = {k: torch.rand(v.lower.shape, generator=g) for k, v in pre.items()} if with_beta else None
    ref32, ga32, gb32 = _oracle_grads(w, alpha, beta, splits)
    ref64, ga64, gb64 = _oracle_grads(w, alpha, beta, splits, dtype=torch.float64)
    wd = wl.to_device(w, dev)
    sd = None if splits is None else {k: v.to(dev) for k, v in splits.items()}
    bounds, ga, gb = hab.lower_bound_gradients(
        wd.module, wd.spec, linear_spec_C=wd.C, relu_alpha={k: v.to(dev) for k, v in alpha.items()},
        relu_beta=None if beta is None else {k: v.to(dev) for k, v in beta.items()}, relu_split_state=sd)
    torch.cuda.synchronize()
    assert_parity(bounds.lower, ref32.lower, ref64.lower, f"{kind} lower")
    allow = None
    if beta is None:
        allow, nties = _sign_tie_allowance(parity.to_float64(w), {k: v.double() for k, v in alpha.items()},
                                           per_batch=True)
        announce(f"{kind}: {nties} input-layer coefficients within fp32 rounding of zero")
    assert set(ga.keys()) == set(ga32.keys())
    for k in ga32:
        _grad_close(ga[k], ga32[k], ga64[k], f"{kind} dL/dalpha[{k}]", None if allow is None else allow[k])
    if gb32 is not None:
        for k in gb32:
            _grad_close(gb[k], gb32[k], gb64[k], f"{kind} dL/dbeta[{k}]")


@pytest.mark.parametrize("kind", ["residual_mlp", "channel_concat_cnn"])
def test_dag_alpha_crown_matches_oracle(kind):
    """Per-domain alpha from the CROWN relaxation, 10 Adam steps (the C4 recipe) on a DAG task."""
    dev = device()
    announce(f"DAG alpha-CROWN {kind}, 10 steps")
    w = wl.make_dag(kind, seed=9, batch=4, eps=0.03, blocks=2)
    wd = wl.to_device(w, dev)
    bounds, alpha, _beta, _st = hab.run_alpha_crown_from_crown_init(wd.module, wd.spec, linear_spec_C=wd.C,
                                                                    steps=10, lr=0.1)
    torch.cuda.synchronize()
    _env, pre = cr.forward_ibp_trace(w.module, w.spec)
    init = ab.adaptive_alpha_init(pre)
    ref = ab.run_alpha_beta_crown(w.module, w.spec, linear_spec_C=w.C, steps=10, lr=0.1, warm_start_alpha=init,
                                  per_batch_params=True)[0]
    crown = cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C)
    # Adam trajectories of two fp32 runs drift by rounding: 1e-4 relative, as for C4
    assert_bounds_close(bounds.lower, ref.lower, f"{kind} alpha lower", rtol=1e-4, atol=1e-4)
    assert_bounds_close(bounds.upper, ref.upper, f"{kind} alpha upper", rtol=1e-4, atol=1e-4)
    assert bool((bounds.lower.cpu() >= crown.lower - 1e-4 * crown.lower.abs() - 1e-4).all())


def test_dag_alpha_beta_crown_with_splits_matches_oracle():
    """alpha-beta-CROWN (per-domain parameters, split multipliers) on the residual MLP."""
    dev = device()
    announce("DAG alpha-beta-CROWN residual_mlp with splits, 8 steps")
    g = torch.Generator().manual_seed(33)
    w = wl.make_dag("residual_mlp", seed=10, batch=4, eps=0.03, blocks=2)
    splits = _feasible_splits(w, g)
    wd = wl.to_device(w, dev)
    bounds, _a, _b, _st = hab.run_alpha_beta_crown_mlp(
        wd.module, wd.spec, linear_spec_C=wd.C, relu_split_state={k: v.to(dev) for k, v in splits.items()},
        steps=8, lr=0.2, per_batch_params=True)
    torch.cuda.synchronize()
    ref = ab.run_alpha_beta_crown(w.module, w.spec, linear_spec_C=w.C, relu_split_state=splits, steps=8, lr=0.2,
                                  per_batch_params=True)[0]
    assert_bounds_close(bounds.lower, ref.lower, "alpha-beta lower", rtol=1e-4, atol=1e-4)
    assert_bounds_close(bounds.upper, ref.upper, "alpha-beta upper", rtol=1e-4, atol=1e-4)


DAG_BAB = {
    "ab_e006_s11": (0.06, 11, dict(max_nodes=40, oracle="alpha_beta", node_batch_size=8, alpha_steps=10)),
    "ab_e006_s12": (0.06, 12, dict(max_nodes=40, oracle="alpha_beta", node_batch_size=8, alpha_steps=10)),
    "alpha_e003_s12": (0.03, 12, dict(max_nodes=20, oracle="alpha", node_batch_size=1, alpha_steps=10)),
}


@pytest.mark.parametrize("tag", list(DAG_BAB))
def test_dag_bab_search_matches_oracle(tag):
    """solve_bab_mlp on a residual MLP: the whole search (statuses, node counts, rounds,
    queue) identical to the oracle's, best bounds within rtol 1e-4."""
    from boundflow_amd import bab as hbab
    from oracle import bab_ref
    dev = device()
    eps, seed, kw = DAG_BAB[tag]
    announce(f"DAG solve_bab_mlp {tag}")
    w = wl.make_dag("residual_mlp", seed=seed, batch=4, eps=eps, n_in=8, hidden=12, n_out=4, blocks=1)
    cfg = dict(use_branch_hint=True, alpha_lr=0.2, alpha_init=0.5, beta_init=0.0, threshold=0.0, tol=1e-6, **kw)
    ref = bab_ref.solve_bab_mlp(w.module, w.spec, linear_spec_C=w.C, config=cfg)
    wd = wl.to_device(w, dev)
    r = hbab.solve_bab_mlp(wd.module, wd.spec, linear_spec_C=wd.C, config=hbab.BabConfig(**kw))
    per = r.per_example
    announce(f"  statuses {[p.status for p in per]} visited {[p.nodes_visited for p in per]} rounds {r.batch_rounds}")
    assert r.status == ref["status"]
    assert [p.status for p in per] == ref["per_status"]
    assert [p.nodes_visited for p in per] == ref["per_visited"]
    assert [p.nodes_evaluated for p in per] == ref["per_evaluated"]
    assert [p.nodes_expanded for p in per] == ref["per_expanded"]
    assert (r.max_queue, r.batch_rounds) == (ref["max_queue"], ref["batch_rounds"])
    import numpy as np
    np.testing.assert_allclose([p.best_lower for p in per], ref["per_best_lower"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose([p.best_upper for p in per], ref["per_best_upper"], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("net", ["c1", "c3", "residual_mlp", "channel_concat_cnn"])
def test_relu_influence_matches_oracle(net):
    """run_crown_ibp_mlp_with_relu_influence_from_forward_trace (crown_ibp.py:2201-2241): the
    objective bounds at the contract and each ReLU's influence (max over specs of the
    coefficient magnitudes, bf_rows_abs_max) within the rounding of the coefficients."""
    dev = device()
    announce(f"ReLU objective influence {net}")
    if net == "c1":
        w = wl.make_c1(batch=8)
    elif net == "c3":
        w = wl.make_c3(batch=4)
    else:
        w = wl.make_dag(net, seed=5, batch=3, eps=0.03, blocks=2)
    wd = wl.to_device(w, dev)
    tr = hc.forward_ibp_trace(wd.module, wd.spec)
    got, infl = hc.run_crown_ibp_mlp_with_relu_influence_from_forward_trace(
        wd.module, wd.spec, interval_env=tr.interval_env, relu_pre=tr.relu_pre, linear_spec_C=wd.C)
    torch.cuda.synchronize()
    env, pre = cr.forward_ibp_trace(w.module, w.spec)
    ref_infl = {}
    ref = cr.crown_backward_from_trace(w.module, w.spec, interval_env=env, relu_pre=pre, linear_spec_C=w.C,
                                       relu_influence_out=ref_infl)
    w64 = parity.to_float64(w)
    env64, pre64 = cr.forward_ibp_trace(w64.module, w64.spec)
    ref64 = cr.crown_backward_from_trace(w64.module, w64.spec, interval_env=env64, relu_pre=pre64,
                                         linear_spec_C=w64.C)
    assert_parity(got.lower, ref.lower, ref64.lower, f"{net} lower")
    assert_parity(got.upper, ref.upper, ref64.upper, f"{net} upper")
    assert list(infl) == list(pre) and set(ref_infl) == set(pre)   # in relu_pre order, as the reference returns it
    for k in ref_infl:
        scale = float(ref_infl[k].abs().max())
        assert_bounds_close(infl[k], ref_infl[k], f"{net} influence[{k}]", rtol=1e-5, atol=1e-6 * scale)
