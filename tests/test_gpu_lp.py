"""HIP parity of L2 and L1 input balls (LpBallPerturbation p=2, p=1) against the oracle.

The input set enters in two places (boundflow/runtime/perturbation.py:102-222):
the first linear layer's IBP box (eps times the dual norm of each weight row:
the L2 norm for an L2 ball, max |w| for an L1 ball) and the final
concretization of the backward coefficient (the same dual norm of each
coefficient row); a first conv layer takes the ball's bounding box in the
forward pass (crown_ibp.py:125-178).  Each path that concretizes is covered:
the fused input region of an MLP, the relaxation-epilogue contraction, every
intermediate bound, a CNN's fused input conv, the DAG backward, and the IBP
task executor.  The alpha/beta reverse pass seeds the concretization's gradient with
the dual norm's derivative (y / ||y||_2, or sign(y) on the maxima of |y|), checked
against autograd through the oracle; alpha-CROWN, alpha-beta-CROWN with splits,
the first-layer certificate and whole BaB searches run over the balls too.  The
oracle's L1/L2 arithmetic is pinned in tests/test_oracle_lp.py and
tests/test_oracle_certificate.py.
"""

import pytest
import torch

from boundflow_amd import alpha_beta as hab
from boundflow_amd import bab as hbab
from boundflow_amd import crown as hc
from boundflow_amd import task_executor as te
from boundflow_amd import workloads as wl
from boundflow_amd.spec import InputSpec, LpBallPerturbation
from oracle import alpha_beta_ref as ab
from oracle import crown_ref as cr
from oracle import parity
from oracle import task_ibp_ref as ti
from tests.gpu_util import announce, assert_bounds_close, assert_parity, assert_verdicts, device
from tests.test_gpu_conv_alpha import _grad_close, _oracle_grads
from tests.test_gpu_crown_dag import _feasible_splits
from tests.test_oracle_certificate import LP_KATS, first_layer_module, lp_spec

pytestmark = pytest.mark.gpu

# radii that leave a mix of stable and unstable ReLUs on the test networks
EPS = {"mlp": {2: 0.3, 1: 1.0}, "cnn": {2: 0.02, 1: 0.03}, "dag": {2: 0.08, 1: 0.2}, "c5": {2: 0.1, 1: 0.5},
       "c4": {2: 0.01, 1: 0.01}}


def _lp(w, p, eps, C=None):
    spec = InputSpec(value_name=w.spec.value_name, center=w.spec.center,
                     perturbation=LpBallPerturbation(p=p, eps=eps))
    return wl.Workload(w.name, w.module, spec, w.C if C is None else C, w.labels, {})


def _crown_check(w, dev, what):
    wd = wl.to_device(w, dev)
    got = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
    torch.cuda.synchronize()
    ref = cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C)
    w64 = parity.to_float64(w)
    ref64 = cr.run_crown_ibp(w64.module, w64.spec, linear_spec_C=w64.C)
    assert_parity(got.lower, ref.lower, ref64.lower, f"{what} lower")
    assert_parity(got.upper, ref.upper, ref64.upper, f"{what} upper")
    assert_verdicts(got.lower, ref.lower, ref64.lower, what)
    # a ball's bound is looser than the point's value and not absurdly so
    assert bool((got.lower <= got.upper).all())


@pytest.mark.parametrize("p", [2, 1])
def test_crown_mlp_lp_matches_oracle(p):
    dev = device()
    announce(f"run_crown_ibp_mlp L{p} ball, C1 network, 16 inputs")
    _crown_check(_lp(wl.make_c1(batch=16), p, EPS["mlp"][p]), dev, f"C1 L{p}")


@pytest.mark.parametrize("p", [2, 1])
def test_crown_epilogue_path_lp_matches_oracle(p, monkeypatch):
    """20 spec rows per domain on the relaxation-epilogue contraction at every hidden
    layer, the input layer's coefficient concretized by bf_crown_linear_concretize."""
    dev = device()
    monkeypatch.setattr(hc, "EPILOGUE_MIN_M", 0)
    announce(f"CROWN L{p} ball on the relaxation-epilogue path")
    B, S = 12, 20
    w = wl.make_c2(batch=B, width=200, depth=4)
    C = torch.randn(B, S, 10, generator=torch.Generator().manual_seed(23))
    _crown_check(_lp(w, p, 0.05 if p == 2 else 0.2, C), dev, f"epilogue L{p}")


@pytest.mark.parametrize("p", [2, 1])
def test_all_intermediate_lp_matches_oracle(p):
    """Every intermediate bound by CROWN (each one an input concretization over the ball)."""
    dev = device()
    announce(f"all-intermediate CROWN L{p} ball, C2 network, 4 inputs")
    w = _lp(wl.subset(wl.make_c2(), 4), p, 0.05 if p == 2 else 0.2)
    wd = wl.to_device(w, dev)
    final, pre = hc.run_crown_all_intermediate(wd.module, wd.spec, linear_spec_C=wd.C)
    torch.cuda.synchronize()
    w64 = parity.to_float64(w)
    ref64, pre64 = cr.run_crown_all_intermediate(w64.module, w64.spec, linear_spec_C=w64.C)
    ref32, _ = cr.run_crown_all_intermediate(w.module, w.spec, linear_spec_C=w.C)
    for name, st in pre.items():
        assert_bounds_close(st.lower, pre64[name].lower, f"L{p} pre {name} lower", rtol=1e-5, atol=1e-5)
        assert_bounds_close(st.upper, pre64[name].upper, f"L{p} pre {name} upper", rtol=1e-5, atol=1e-5)
    assert_parity(final.lower, ref32.lower, ref64.lower, f"all-intermediate L{p} lower")
    assert_parity(final.upper, ref32.upper, ref64.upper, f"all-intermediate L{p} upper")


@pytest.mark.parametrize("p", [2, 1])
def test_crown_cnn_lp_matches_oracle(p):
    """The C3 CNN: bounding-box IBP through the input conv, the backward's input conv
    reduced to the ball's norm in the fused input-layer kernel."""
    dev = device()
    announce(f"run_crown_ibp_mlp L{p} ball, C3 network, 8 inputs")
    _crown_check(_lp(wl.make_c3(batch=8), p, EPS["cnn"][p]), dev, f"C3 L{p}")


@pytest.mark.parametrize("kind", wl.DAG_KINDS)
@pytest.mark.parametrize("p", [2, 1])
def test_dag_crown_lp_matches_oracle(kind, p):
    dev = device()
    announce(f"DAG CROWN {kind} L{p} ball")
    _crown_check(_lp(wl.make_dag(kind), p, EPS["dag"][p]), dev, f"{kind} L{p}")


@pytest.mark.parametrize("p", [2, 1])
def test_task_executor_ibp_lp_matches_oracle(p):
    """HipTaskExecutor.run_ibp: the first linear layer concretized over the ball
    (bf_ibp_linear input kinds 2 and 3), every later layer interval arithmetic."""
    dev = device()
    announce(f"HipTaskExecutor.run_ibp L{p} ball, C1 network")
    w = _lp(wl.make_c1(batch=16), p, EPS["mlp"][p])
    wd = wl.to_device(w, dev)
    out = te.HipTaskExecutor().run_ibp(wd.module, wd.spec)
    torch.cuda.synchronize()
    w64 = parity.to_float64(w)
    ref64 = ti.run_ibp(w64.module, w64.spec)
    ref = ti.run_ibp(w.module, w.spec)
    assert_parity(out.lower, ref.lower, ref64.lower, f"IBP L{p} lower")
    assert_parity(out.upper, ref.upper, ref64.upper, f"IBP L{p} upper")


def _grad_case(case, p):
    g = torch.Generator().manual_seed(41 + p)
    if case.startswith("mlp"):
        w = _lp(wl.subset(wl.make_c5(depth=2, label_mode="predicted"), 12), p, EPS["c5"][p])
    elif case == "cnn":
        w = _lp(wl.subset(wl.make_c4(), 3), p, EPS["c4"][p])
    else:
        kind = {"dag": "residual_mlp", "dag_cnn": "channel_concat_cnn"}[case]
        w = _lp(wl.make_dag(kind, seed=8, batch=3, eps=0.03, blocks=2), p, EPS["dag"][p])
    beta_on = case in ("mlp", "mlp_epilogue", "dag")
    splits = _feasible_splits(w, g) if beta_on else None
    _env, pre = cr.forward_ibp_trace(w.module, w.spec, relu_split_state=splits)
    alpha = {k: torch.rand(v.lower.shape, generator=g) for k, v in pre.items()}
    beta = {k: torch.rand(v.lower.shape, generator=g) for k, v in pre.items()} if beta_on else None
    return w, splits, alpha, beta


@pytest.mark.parametrize("case", ["mlp", "mlp_epilogue", "cnn", "dag", "dag_cnn"])
@pytest.mark.parametrize("p", [2, 1])
def test_lp_lower_bound_gradients_match_autograd(case, p, monkeypatch):
    """dL/dalpha and dL/dbeta for L = -sum_d mean_s lb over an L2 / L1 ball: the
    chain's fused input region (and, with mlp_epilogue, the relaxation-epilogue path's
    plain concretization), the CNN's fused input conv, and the DAG reverse pass."""
    dev = device()
    announce(f"L{p} alpha/beta gradient pass vs autograd: {case}")
    if case == "mlp_epilogue":
        monkeypatch.setattr(hc, "EPILOGUE_MIN_M", 0)
    w, splits, alpha, beta = _grad_case(case, p)
    ref32, ga32, gb32 = _oracle_grads(w, alpha, beta, splits)
    ref64, ga64, gb64 = _oracle_grads(w, alpha, beta, splits, dtype=torch.float64)
    wd = wl.to_device(w, dev)
    sd = None if splits is None else {k: v.to(dev) for k, v in splits.items()}
    bounds, ga, gb = hab.lower_bound_gradients(
        wd.module, wd.spec, linear_spec_C=wd.C, relu_alpha={k: v.to(dev) for k, v in alpha.items()},
        relu_beta=None if beta is None else {k: v.to(dev) for k, v in beta.items()}, relu_split_state=sd)
    torch.cuda.synchronize()
    assert_parity(bounds.lower, ref32.lower, ref64.lower, f"L{p} {case} lower")
    assert set(ga.keys()) == set(ga32.keys())
    for k in ga32:
        _grad_close(ga[k], ga32[k], ga64[k], f"L{p} {case} dL/dalpha[{k}]")
    if gb32 is not None:
        for k in gb32:
            _grad_close(gb[k], gb32[k], gb64[k], f"L{p} {case} dL/dbeta[{k}]")


@pytest.mark.parametrize("net", ["c1", "dag"])
@pytest.mark.parametrize("p", [2, 1])
def test_lp_alpha_crown_matches_oracle(net, p):
    """alpha-CROWN from the CROWN slopes, 10 Adam steps (the C4 recipe), over an L2 / L1
    ball: the final bounds at the contract, a domain outside it traced step by step
    (oracle/trajectory.py); never looser than CROWN.  On the C1 network the oracle's
    trajectory is the reference's own (fixture lp_reference_p{p}, pinned in
    tests/test_oracle_lp.py), and the HIP bounds are compared with the fixture too."""
    from oracle import trajectory as tt
    from tests.golden_util import load, lp_case, t
    dev = device()
    announce(f"L{p} alpha-CROWN {net}, 10 steps")
    if net == "c1":
        w = lp_case("alpha", p)
    else:
        w = _lp(wl.make_dag("residual_mlp", seed=9, batch=4, eps=0.03, blocks=2), p, EPS["dag"][p])
    wd = wl.to_device(w, dev)
    hrec = []
    bounds, best_alpha, _beta, _st = hab.run_alpha_crown_from_crown_init(wd.module, wd.spec, linear_spec_C=wd.C,
                                                                         steps=10, lr=0.1, record=hrec)
    torch.cuda.synchronize()
    _env, pre = cr.forward_ibp_trace(w.module, w.spec)
    srec = []
    ref = ab.run_alpha_beta_crown(w.module, w.spec, linear_spec_C=w.C, steps=10, lr=0.1,
                                  warm_start_alpha=ab.adaptive_alpha_init(pre), per_batch_params=True,
                                  record=srec)[0]
    crown = cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C)

    def fp64_lower(rows):
        w64 = parity.to_float64(tt.sub_workload(w, rows))
        _e64, pre64 = cr.forward_ibp_trace(w64.module, w64.spec)
        return ab.run_alpha_beta_crown(w64.module, w64.spec, linear_spec_C=w64.C, steps=10, lr=0.1,
                                       warm_start_alpha=ab.adaptive_alpha_init(pre64), per_batch_params=True)[0].lower

    summary = tt.trace_run(w, hrec, srec, bounds.lower.cpu(), ref.lower, 0.1, what=f"L{p} {net} alpha",
                           sample=range(w.batch), got_upper=bounds.upper.cpu(), ref_upper=ref.upper,
                           best_alpha={n: v.cpu() for n, v in best_alpha.items()}, fp64_lower=fp64_lower,
                           log=announce)
    announce(f"  trace: {summary}")
    assert bool((bounds.lower.cpu() >= crown.lower - 1e-4 * crown.lower.abs() - 1e-4).all())
    if net == "c1":
        g = load(f"lp_reference_p{p}")
        assert torch.allclose(ref.lower, t(g["alpha_lower"]), rtol=1e-5, atol=1e-6)
        assert torch.allclose(ref.upper, t(g["alpha_upper"]), rtol=1e-5, atol=1e-6)
        out = tt.domains_outside(torch.cat([bounds.lower.cpu(), bounds.upper.cpu()], 1),
                                 torch.cat([t(g["alpha_lower"]), t(g["alpha_upper"])], 1))
        announce(f"  vs the reference fixture: domains outside the contract {out} (traced above against the "
                 f"oracle, whose trajectory is the reference's)")


@pytest.mark.parametrize("p", [2, 1])
def test_lp_alpha_beta_crown_with_splits_matches_oracle(p):
    """alpha-beta-CROWN with splits over an L2 / L1 ball: final bounds at the contract, a
    domain outside it traced step by step (oracle/trajectory.py)."""
    from oracle import trajectory as tt
    dev = device()
    announce(f"L{p} alpha-beta-CROWN residual_mlp with splits, 8 steps")
    g = torch.Generator().manual_seed(33)
    w = _lp(wl.make_dag("residual_mlp", seed=10, batch=4, eps=0.03, blocks=2), p, EPS["dag"][p])
    splits = _feasible_splits(w, g)
    w = wl.Workload(w.name, w.module, w.spec, w.C, w.labels, {"splits": splits})
    wd = wl.to_device(w, dev)
    hrec = []
    bounds, best_alpha, _b, _st = hab.run_alpha_beta_crown_mlp(
        wd.module, wd.spec, linear_spec_C=wd.C, relu_split_state={k: v.to(dev) for k, v in splits.items()},
        steps=8, lr=0.2, per_batch_params=True, record=hrec)
    torch.cuda.synchronize()
    srec = []
    ref = ab.run_alpha_beta_crown(w.module, w.spec, linear_spec_C=w.C, relu_split_state=splits, steps=8, lr=0.2,
                                  per_batch_params=True, record=srec)[0]

    def fp64_lower(rows):
        w64 = parity.to_float64(tt.sub_workload(w, rows))
        return ab.run_alpha_beta_crown(w64.module, w64.spec, linear_spec_C=w64.C,
                                       relu_split_state=w64.extra["splits"], steps=8, lr=0.2,
                                       per_batch_params=True)[0].lower

    summary = tt.trace_run(w, hrec, srec, bounds.lower.cpu(), ref.lower, 0.2, what=f"L{p} alpha-beta",
                           sample=range(w.batch), got_upper=bounds.upper.cpu(), ref_upper=ref.upper,
                           best_alpha={n: v.cpu() for n, v in best_alpha.items()}, fp64_lower=fp64_lower,
                           log=announce)
    announce(f"  trace: {summary}")


@pytest.mark.parametrize("p", [2, 1])
def test_hip_matches_lp_reference_fixtures(p):
    """The HIP path against the reference's own runs over an L2 / L1 ball (fixture
    lp_reference_p{p}): CROWN on the C1 MLP and the C3 CNN at the contract
    (fp64-explained), the first-layer certificate's flags and max_value on the
    geometric known answers and on 48 C5 first-layer nodes, and a whole BaB search."""
    import numpy as np
    from boundflow_amd.ir import BFTaskModule
    from boundflow_amd.split_certificate import split_certificate
    from tests.golden_util import LP_BAB, load, lp_case, lp_cert_nodes, t, workload_checksum
    dev = device()
    announce(f"HIP vs the reference's L{p} runs")
    g = load(f"lp_reference_p{p}")
    for kind in ("mlp", "cnn"):
        w = lp_case(kind, p)
        assert workload_checksum(w) == str(g[f"crown_{kind}_checksum"])
        wd = wl.to_device(w, dev)
        got = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
        w64 = parity.to_float64(w)
        ref64 = cr.run_crown_ibp(w64.module, w64.spec, linear_spec_C=w64.C)
        assert_parity(got.lower, t(g[f"crown_{kind}_lower"]), ref64.lower, f"L{p} {kind} lower vs reference")
        assert_parity(got.upper, t(g[f"crown_{kind}_upper"]), ref64.upper, f"L{p} {kind} upper vs reference")
    for name, (Wk, bk, sk, _e) in LP_KATS.items():
        m = first_layer_module(torch.tensor(Wk), torch.tensor(bk))
        md = BFTaskModule(tasks=m.tasks, entry_task_id=m.entry_task_id,
                          bindings={"params": {k: v.to(dev) for k, v in m.params.items()}})
        val = torch.empty(1, device=dev)
        flag = split_certificate(md, lp_spec(p, torch.zeros(1, 2, device=dev)),
                                 {"h1": torch.tensor([sk], dtype=torch.int8, device=dev)}, {"h1": (len(bk),)},
                                 max_out=val).cpu().tolist()[0]
        assert flag == int(g[f"kat_{name}_flag"]), name
        if flag:
            ref = float(g[f"kat_{name}_value"])
            assert abs(float(val.cpu()[0]) - ref) <= 1e-5 * abs(ref) + 1e-5, (name, float(val.cpu()[0]), ref)
    w = lp_case("cert_c5", p)
    name, rows = lp_cert_nodes(w, p)
    wd = wl.to_device(w, dev)
    vals = torch.empty(int(rows.shape[0]), device=dev)
    flags = split_certificate(wd.module, wd.spec, {name: rows.to(dev)}, {n: (256,) for n in wl.relu_input_names(
        w.module)}, max_out=vals).cpu()
    announce(f"  C5 first-layer nodes closed: hip {int(flags.sum())}, reference {int(g['cert_c5_flag'].sum())}")
    assert flags.tolist() == g["cert_c5_flag"].tolist()
    closed = flags.bool().numpy()
    if closed.any():
        ref = g["cert_c5_value"][closed]
        np.testing.assert_allclose(vals.cpu().numpy()[closed], ref, rtol=1e-4, atol=1e-5)
    w = lp_case("bab", p)
    wd = wl.to_device(w, dev)
    r = hbab.solve_bab_mlp(wd.module, wd.spec, linear_spec_C=wd.C, config=hbab.BabConfig(**LP_BAB[p][1]))
    per = r.per_example
    code = {"proven": 0, "unsafe": 1, "unknown": 2}
    announce(f"  BaB statuses {[q.status for q in per]} visited {[q.nodes_visited for q in per]}")
    assert [code[q.status] for q in per] == g["bab_per_status"].tolist()
    assert [q.nodes_visited for q in per] == g["bab_per_visited"].tolist()
    assert [q.nodes_evaluated for q in per] == g["bab_per_evaluated"].tolist()
    assert [q.nodes_expanded for q in per] == g["bab_per_expanded"].tolist()
    assert (r.max_queue, r.batch_rounds) == (int(g["bab_max_queue"]), int(g["bab_batch_rounds"]))


@pytest.mark.parametrize("p", ["inf", 2, 1])
@pytest.mark.parametrize("name", list(LP_KATS))
def test_lp_certificate_known_answers(name, p):
    """The first-layer certificate (bf_split_certificate) over Linf, L2 and L1 balls on the
    geometric known answers, and run_alpha_beta_crown_mlp's infeasible result."""
    from boundflow_amd.ir import BFTaskModule
    from boundflow_amd.split_certificate import split_certificate
    dev = device()
    announce(f"split certificate L{p} KAT {name}")
    W, b, s, expect = LP_KATS[name]
    m = first_layer_module(torch.tensor(W), torch.tensor(b))
    md = BFTaskModule(tasks=m.tasks, entry_task_id=m.entry_task_id,
                      bindings={"params": {k: v.to(dev) for k, v in m.params.items()}})
    spec = lp_spec(p, torch.zeros(1, 2, device=dev))
    split = {"h1": torch.tensor([s], dtype=torch.int8, device=dev)}
    flags = split_certificate(md, spec, split, {"h1": (len(b),)}).cpu().tolist()
    ibp_closes = False
    try:
        cr.forward_ibp_trace(m, lp_spec(p, torch.zeros(1, 2)), relu_split_state={"h1": split["h1"].cpu()})
    except ValueError:
        ibp_closes = True
    assert flags == [1 if expect[p] else 0] or ibp_closes
    _bounds, _alpha, _beta, stats = hab.run_alpha_beta_crown_mlp(md, spec, relu_split_state=split, steps=0)
    assert stats.feasibility == ("infeasible" if expect[p] else "unknown")
    # the reference's stand-alone check (alpha_beta_crown.py:109-142) sees the certificate alone
    chk = hab.check_first_layer_infeasible_split(md, spec, relu_split_state=split)
    assert chk.feasibility == ("infeasible" if flags == [1] else "unknown")


@pytest.mark.parametrize("p", [2, 1])
def test_lp_certificate_matches_oracle_on_c5_first_layer(p):
    from tests.test_gpu_certificate import _random_nodes, _row_spec
    from boundflow_amd.split_certificate import split_certificate
    dev = device()
    announce(f"split certificate vs oracle, C5 first layer, 48 nodes, L{p}")
    g = torch.Generator().manual_seed(4 + p)
    w = _lp(wl.make_c5(domains=48), p, {2: 0.5, 1: 2.0}[p])
    name, rows = _random_nodes(w, g, 48, 12)
    shapes = {n: (256,) for n in wl.relu_input_names(w.module)}
    wd = wl.to_device(w, dev)
    got = split_certificate(wd.module, wd.spec, {name: rows.to(dev)}, shapes).cpu().tolist()
    ref = [int(ab.split_certificate(w.module, _row_spec(w.spec, r), {name: rows[r:r + 1]})[0]) for r in range(48)]
    announce(f"  infeasible nodes: hip {sum(got)}, oracle {sum(ref)}")
    assert got == ref


BAB_LP = {
    "alpha_beta_l2": (2, 0.1, dict(max_nodes=40, oracle="alpha_beta", node_batch_size=8, alpha_steps=10)),
    "alpha_l1": (1, 0.25, dict(max_nodes=20, oracle="alpha", node_batch_size=1, alpha_steps=10)),
}


@pytest.mark.parametrize("tag", list(BAB_LP))
def test_lp_bab_search_matches_oracle(tag):
    """solve_bab_mlp over an L2 / L1 ball: the whole search identical to the oracle's."""
    from oracle import bab_ref
    dev = device()
    p, eps, kw = BAB_LP[tag]
    announce(f"solve_bab_mlp {tag}")
    base = wl.make_dag("residual_mlp", seed=12, batch=4, eps=0.03, n_in=8, hidden=12, n_out=4, blocks=1)
    w = _lp(base, p, eps)
    cfg = dict(use_branch_hint=True, alpha_lr=0.2, alpha_init=0.5, beta_init=0.0, threshold=0.0, tol=1e-6, **kw)
    ref = bab_ref.solve_bab_mlp(w.module, w.spec, linear_spec_C=w.C, config=cfg)
    wd = wl.to_device(w, dev)
    r = hbab.solve_bab_mlp(wd.module, wd.spec, linear_spec_C=wd.C, config=hbab.BabConfig(**kw))
    per = r.per_example
    announce(f"  statuses {[q.status for q in per]} visited {[q.nodes_visited for q in per]} "
             f"rounds {r.batch_rounds}; oracle {ref['per_status']} {ref['per_visited']}")
    assert [q.status for q in per] == ref["per_status"]
    assert [q.nodes_visited for q in per] == ref["per_visited"]
    assert [q.nodes_evaluated for q in per] == ref["per_evaluated"]
    assert [q.nodes_expanded for q in per] == ref["per_expanded"]
    assert (r.max_queue, r.batch_rounds) == (ref["max_queue"], ref["batch_rounds"])
    import numpy as np
    np.testing.assert_allclose([q.best_lower for q in per], ref["per_best_lower"], rtol=1e-4, atol=1e-5)


def test_certificate_record_and_state_objects():
    """The reference's result types: the L2 three-directions query closes with a
    certificate whose max_value is negative (tests/test_phase6f_alpha_beta_crown_pr1.py:96-118);
    alpha/beta come back as AlphaState / BetaState (dicts with alpha_by_relu_input /
    beta_by_relu_input) and are taken back as warm starts in either form."""
    from types import SimpleNamespace
    dev = device()
    announce("certificate record and AlphaState/BetaState round trip")
    W, b, s, _expect = LP_KATS["three_directions"]
    m = first_layer_module(torch.tensor(W), torch.tensor(b))
    from boundflow_amd.ir import BFTaskModule
    md = BFTaskModule(tasks=m.tasks, entry_task_id=m.entry_task_id,
                      bindings={"params": {k: v.to(dev) for k, v in m.params.items()}})
    spec = lp_spec(2, torch.zeros(1, 2, device=dev))
    split = {"h1": torch.tensor([s], dtype=torch.int8, device=dev)}
    _b, alpha, beta, stats = hab.run_alpha_beta_crown_mlp(md, spec, relu_split_state=split, steps=0, lr=0.2)
    assert stats.feasibility == "infeasible" and stats.infeasible_certificate is not None
    assert float(stats.infeasible_certificate["max_value"]) < 0.0
    chk = hab.check_first_layer_infeasible_split(md, spec, relu_split_state=split)
    assert chk.feasibility == "infeasible" and float(chk.infeasible_certificate["max_value"]) < 0.0
    assert isinstance(alpha, hab.AlphaState) and isinstance(beta, hab.BetaState)
    w = wl.to_device(_lp(wl.make_c1(batch=4), 2, EPS["mlp"][2]), dev)
    b1, a1, st1 = hab.run_alpha_crown_mlp(w.module, w.spec, linear_spec_C=w.C, steps=3, lr=0.1)
    assert isinstance(a1, hab.AlphaState) and a1.alpha_by_relu_input is a1
    clone = a1.detach_clone()
    for warm in (clone, SimpleNamespace(alpha_by_relu_input=dict(clone)), dict(clone)):
        b2, _a2, _s2 = hab.run_alpha_crown_mlp(w.module, w.spec, linear_spec_C=w.C, steps=0, lr=0.1, warm_start=warm)
        # zero steps from the best alpha of the first run: its bound again
        assert torch.allclose(b2.lower, b1.lower, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("p", ["inf", 2, 1])
def test_task_executor_per_sample_weights_over_balls(p):
    """HipTaskExecutor.run_ibp with a rank-3 linear weight W [B, O, I] applied to the input
    ball (perturbation.py:146-173): the ball's dual norm of each W[b] row."""
    from boundflow_amd.ir import BFTaskModule, BoundTask, TaskKind, TaskOp
    dev = device()
    announce(f"HipTaskExecutor per-sample weights, L{p} ball")
    g = torch.Generator().manual_seed(61)
    B, O, I = 5, 7, 33
    W = torch.randn(B, O, I, generator=g)
    bias = torch.randn(O, generator=g)
    x0 = torch.randn(B, I, generator=g)
    task = BoundTask(task_id="t0", kind=TaskKind.INTERVAL_IBP,
                     ops=[TaskOp("linear", "l", ["input", "W", "b"], ["out"])], input_values=["input"],
                     output_values=["out"])

    def mod(dev_):
        return BFTaskModule(tasks=[task], entry_task_id="t0", bindings={"params": {"W": W.to(dev_), "b": bias.to(dev_)}})

    got = te.HipTaskExecutor().run_ibp(mod(dev), lp_spec(p, x0.to(dev), 0.2))
    torch.cuda.synchronize()
    ref = ti.run_ibp(mod("cpu"), lp_spec(p, x0, 0.2))
    ref64 = ti.run_ibp(BFTaskModule(tasks=[task], entry_task_id="t0",
                                    bindings={"params": {"W": W.double(), "b": bias.double()}}),
                       lp_spec(p, x0.double(), 0.2))
    assert_parity(got.lower, ref.lower, ref64.lower, f"per-sample L{p} lower")
    assert_parity(got.upper, ref.upper, ref64.upper, f"per-sample L{p} upper")
