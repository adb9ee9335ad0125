"""The first-layer split certificate on the device (bf_split_certificate, one
workgroup per node) against the oracle's restatement of the reference
(oracle/alpha_beta_ref.py split_certificate): the reference's known answers,
random halfspace sets in 2-D and on the first layer of the C5 network (784
inputs, Linf and box inputs), and the B==1 path of run_alpha_beta_crown_mlp."""

import pytest
import torch

from boundflow_amd import alpha_beta as hab
from boundflow_amd import workloads as wl
from boundflow_amd.spec import InputSpec
from boundflow_amd.split_certificate import split_certificate
from oracle import alpha_beta_ref as ab
from tests.gpu_util import announce, device
from tests.test_oracle_certificate import KATS, first_layer_module

pytestmark = pytest.mark.gpu


def _to(m, dev):
    from boundflow_amd.ir import BFTaskModule
    return BFTaskModule(tasks=m.tasks, entry_task_id=m.entry_task_id,
                        bindings={"params": {k: v.to(dev) for k, v in m.params.items()}})


@pytest.mark.parametrize("name", list(KATS))
def test_known_answers(name):
    dev = device()
    announce(f"split certificate KAT {name}")
    W, b, s, expect = KATS[name]
    m = first_layer_module(torch.tensor(W), torch.tensor(b))
    md = _to(m, dev)
    spec = InputSpec.linf(value_name="input", center=torch.zeros(1, 2, device=dev), eps=1.0)
    split = {"h1": torch.tensor([s], dtype=torch.int8, device=dev)}
    flags = split_certificate(md, spec, split, {"h1": (len(b),)}).cpu().tolist()
    assert flags == [1 if expect else 0]
    # run_alpha_beta_crown_mlp with one domain returns the reference's infeasible result
    bounds, alpha, beta, stats = hab.run_alpha_beta_crown_mlp(md, spec, relu_split_state=split, steps=0)
    assert stats.feasibility == ("infeasible" if expect else "unknown")
    if expect:
        assert tuple(bounds.lower.shape) == (1, 1) and float(bounds.lower.abs().max()) == 0.0
        assert alpha == {} and beta == {}


def _random_nodes(w, g, count, kmax):
    """Split rows on the first layer's ambiguous neurons: 1..kmax entries of +-1 per node."""
    from oracle import crown_ref as cr
    _env, pre = cr.forward_ibp_trace(w.module, wl.subset(w, 1).spec)
    name = next(iter(pre))
    l, u = pre[name].lower[0], pre[name].upper[0]
    amb = ((l < 0) & (u > 0)).nonzero().flatten()
    n = int(l.numel())
    rows = torch.zeros(count, n, dtype=torch.int8)
    for r in range(count):
        k = int(torch.randint(2, kmax + 1, (1,), generator=g))
        pick = amb[torch.randperm(int(amb.numel()), generator=g)[:k]]
        rows[r, pick] = (torch.randint(0, 2, (int(pick.numel()),), generator=g) * 2 - 1).to(torch.int8)
    return name, rows


@pytest.mark.parametrize("box", [False, True])
def test_matches_oracle_on_c5_first_layer(box):
    dev = device()
    announce(f"split certificate vs oracle, C5 first layer, 48 nodes, box={box}")
    g = torch.Generator().manual_seed(4)
    w = wl.make_c5(domains=48, eps=0.05)
    if box:
        lo = (w.spec.center - 0.05).clamp(0, 1)
        hi = (w.spec.center + 0.05).clamp(0, 1)
        w = wl.Workload("C5box", w.module, InputSpec.box(value_name="input", lower=lo, upper=hi), w.C, w.labels)
    name, rows = _random_nodes(w, g, 48, 12)
    shapes = {n: (256,) for n in wl.relu_input_names(w.module)}
    wd = wl.to_device(w, dev)
    got = split_certificate(wd.module, wd.spec, {name: rows.to(dev)}, shapes).cpu().tolist()
    ref = []
    for r in range(48):
        sub = wl.Workload("one", w.module, _row_spec(w.spec, r), w.C[r:r + 1], w.labels[r:r + 1])
        ref.append(int(ab.split_certificate(w.module, sub.spec, {name: rows[r:r + 1]})[0]))
    announce(f"  infeasible nodes: hip {sum(got)}, oracle {sum(ref)}")
    assert got == ref


def _row_spec(spec, r):
    from boundflow_amd.spec import BoxPerturbation
    p = spec.perturbation
    if isinstance(p, BoxPerturbation):
        return InputSpec.box(value_name=spec.value_name, lower=p.lower[r:r + 1], upper=p.upper[r:r + 1])
    return InputSpec(value_name=spec.value_name, center=spec.center[r:r + 1], perturbation=p)


def test_matches_oracle_on_random_2d_sets():
    dev = device()
    announce("split certificate vs oracle, 64 random 2-D halfspace sets")
    g = torch.Generator().manual_seed(12)
    got, ref = [], []
    for trial in range(64):
        k = int(torch.randint(2, 6, (1,), generator=g))
        W = torch.randn(k, 2, generator=g)
        b = torch.randn(k, generator=g) * 0.5 - 0.3
        s = (torch.randint(0, 2, (1, k), generator=g) * 2 - 1).to(torch.int8)
        m = first_layer_module(W, b)
        spec = InputSpec.linf(value_name="input", center=torch.zeros(1, 2), eps=1.0)
        ref.append(int(ab.split_certificate(m, spec, {"h1": s})[0]))
        sd = InputSpec.linf(value_name="input", center=torch.zeros(1, 2, device=dev), eps=1.0)
        got.append(int(split_certificate(_to(m, dev), sd, {"h1": s.to(dev)}, {"h1": (k,)}).cpu()[0]))
    announce(f"  infeasible: hip {sum(got)}, oracle {sum(ref)}")
    assert sum(ref) >= 4
    assert got == ref
