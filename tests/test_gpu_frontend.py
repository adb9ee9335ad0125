"""The frontend path on the device: nn.Modules imported with ``import_torch`` and
planned with ``plan_interval_ibp_v0`` run on the HIP backend.

* C1 and C3 (chains): the HIP bounds of the planned modules equal the HIP bounds
  of the hand-built workloads bit for bit (same kernels on the same data);
* the reference's DAG frontend nets (residual add, concat): HIP bounds against
  the oracle on the planned module, at the contract;
* a VNNLIB robustness property of a C1 input: box and clause matrix materialised
  from the parsed query, HIP bounds equal to the hand-built C1 query's, and the
  same verdict."""

import pytest
import torch

from boundflow_amd import crown as hc
from boundflow_amd import frontend as fe
from boundflow_amd import vnnlib as vn
from boundflow_amd import workloads as wl
from boundflow_amd.ir import BFTaskModule
from boundflow_amd.spec import InputSpec
from oracle import crown_ref as cr
from oracle import parity
from tests.frontend_models import frontend_nets, sequential_from_chain, vnnlib_c1_property
from tests.gpu_util import announce, assert_parity, device

pytestmark = pytest.mark.gpu


def _on(tm: BFTaskModule, dev) -> BFTaskModule:
    return BFTaskModule(tasks=tm.tasks, entry_task_id=tm.entry_task_id, storage_plan=tm.storage_plan,
                        bindings={**tm.bindings, "params": {k: v.to(dev) for k, v in tm.params.items()}})


@pytest.mark.parametrize("name,n", [("C1", 64), ("C3", 128)])
def test_planned_chain_bounds_equal_hand_built(name, n):
    dev = device()
    announce(f"frontend: planned {name} (B={n}) vs the hand-built workload on the device")
    w = wl.subset(wl.make(name), n)
    example = w.spec.perturbation.lower if name == "C1" else w.spec.center
    tm = fe.plan_interval_ibp_v0(fe.import_torch(sequential_from_chain(w.module), (example[:2],)))
    wd = wl.to_device(w, dev)
    spec = InputSpec(value_name="input", center=wd.spec.center, perturbation=wd.spec.perturbation)
    a = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
    b = hc.run_crown_ibp_mlp(_on(tm, dev), spec, linear_spec_C=wd.C)
    torch.cuda.synchronize()
    assert torch.equal(a.lower, b.lower) and torch.equal(a.upper, b.upper)


@pytest.mark.parametrize("name", ["residual_add", "concat"])
def test_planned_dag_matches_oracle(name):
    dev = device()
    announce(f"frontend: planned DAG net {name} on the device vs the oracle")
    net, _x = frontend_nets()[name]
    g = torch.Generator().manual_seed(5)
    x = torch.rand(6, 1, 2, 2, generator=g)
    prog = fe.import_torch(net, (x[:2],))
    tm = fe.plan_interval_ibp_v0(prog)
    name_in = prog.graph.inputs[0]
    out_dim = int(net(x[:1]).shape[1])
    labels = torch.randint(0, out_dim, (6,), generator=g)
    C = wl.margin_spec(labels, out_dim)
    spec = InputSpec.linf(value_name=name_in, center=x, eps=0.05)
    ref = cr.run_crown_ibp(tm, spec, linear_spec_C=C)
    w64 = wl.Workload("dag", tm, spec, C, labels)
    w64 = parity.to_float64(w64)
    ref64 = cr.run_crown_ibp(w64.module, w64.spec, linear_spec_C=w64.C)
    got = hc.run_crown_ibp_mlp(_on(tm, dev), InputSpec.linf(value_name=name_in, center=x.to(dev), eps=0.05),
                               linear_spec_C=C.to(dev))
    assert_parity(got.lower, ref.lower, ref64.lower, f"{name} lower")
    assert_parity(got.upper, ref.upper, ref64.upper, f"{name} upper")


def test_vnnlib_property_on_the_device():
    dev = device()
    announce("VNNLIB robustness property of C1 input 0 on the device")
    w = wl.to_device(wl.subset(wl.make_c1(), 1), dev)
    q = vn.parse_vnnlib_box_query(vnnlib_c1_property(0), query_id="c1:0")
    t = vn.materialize_vnnlib_box_query(q, input_shape=(784,), device=dev)
    spec = InputSpec.box(value_name="input", lower=t.input_lower, upper=t.input_upper)
    b = hc.run_crown_ibp_mlp(w.module, spec, linear_spec_C=t.linear_spec_c)
    ref = hc.run_crown_ibp_mlp(w.module, w.spec, linear_spec_C=w.C)
    torch.cuda.synchronize()
    assert torch.equal(b.lower, ref.lower) and torch.equal(b.upper, ref.upper)
    assert vn.query_verified(b.lower, t.thresholds) == bool((ref.lower > 0).all())
