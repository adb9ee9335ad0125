"""HIP parity tests of CROWN-IBP on DAG networks (residual add, concat, fan-out):
``run_crown_ibp_mlp`` on a task that is not a chain runs the general backward of
``boundflow_amd.crown_dag`` and must match the oracle (crown_ibp.py:1669-2051),
whose DAG pieces are pinned in tests/test_oracle_dag.py."""

import pytest
import torch

from boundflow_amd import crown as hc
from boundflow_amd import crown_dag
from boundflow_amd import workloads as wl
from oracle import crown_ref as cr
from oracle import parity
from tests.gpu_util import announce, assert_bounds_close, assert_parity, assert_verdicts, device

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
