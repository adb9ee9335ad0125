"""HIP parity of L2 and L1 input balls (LpBallPerturbation p=2, p=1) against the oracle.

The input set enters in two places (boundflow/runtime/perturbation.py:102-222):
the first linear layer's IBP box (eps times the dual norm of each weight row:
the L2 norm for an L2 ball, max |w| for an L1 ball) and the final
concretization of the backward coefficient (the same dual norm of each
coefficient row); a first conv layer takes the ball's bounding box in the
forward pass (crown_ibp.py:125-178).  Each path that concretizes is covered:
the fused input region of an MLP, the relaxation-epilogue contraction, every
intermediate bound, a CNN's fused input conv, the DAG backward, and the IBP
task executor.  The oracle's L1/L2 arithmetic is pinned in
tests/test_oracle_lp.py.
"""

import pytest
import torch

from boundflow_amd import crown as hc
from boundflow_amd import task_executor as te
from boundflow_amd import workloads as wl
from boundflow_amd.spec import InputSpec, LpBallPerturbation
from oracle import crown_ref as cr
from oracle import parity
from oracle import task_ibp_ref as ti
from tests.gpu_util import announce, assert_bounds_close, assert_parity, assert_verdicts, device

pytestmark = pytest.mark.gpu

# radii that leave a mix of stable and unstable ReLUs on the test networks
EPS = {"mlp": {2: 0.5, 1: 1.5}, "cnn": {2: 0.02, 1: 0.03}, "dag": {2: 0.08, 1: 0.2}}


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
