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


def test_conv_first_layer_matches_the_reference_fixture():
    """C3's first conv layer (3x32x32 input: a 12 KB LDS stage; 16x16x16 neurons, the
    Jacobian rows made by the transposed convolution in chunks): 24 nodes with one split
    neuron each, in one launch, against the reference's certificate
    (_is_infeasible_split_first_layer_convex_combo, fixture cert_c3_conv): identical
    flags, the reference's max_value where it closes a node, and the single halfspace's
    maximum (fp64, from the conv's Jacobian row) on every node."""
    from tests.golden_util import load, workload_checksum
    dev = device()
    announce("split certificate, C3 first conv layer, 24 nodes, vs reference fixture")
    g = load("cert_c3_conv")
    w = wl.subset(wl.make_c3(), 8)
    assert workload_checksum(w) == str(g["checksum"])
    ex = torch.as_tensor(g["example"]).long()
    N = int(ex.numel())
    split = torch.zeros(N, 16 * 16 * 16, dtype=torch.int8)
    split[torch.arange(N), torch.as_tensor(g["neuron"]).long()] = torch.as_tensor(g["sign"]).to(torch.int8)
    eps = float(w.spec.perturbation.eps)
    spec = InputSpec.linf(value_name="input", center=w.spec.center[ex].to(dev), eps=eps)
    wd = wl.to_device(w, dev)
    value = torch.empty(N, device=dev)
    flags = split_certificate(wd.module, spec, {"h0": split.reshape(N, 16, 16, 16).to(dev)}, {"h0": (16, 16, 16)},
                              max_out=value).cpu()
    value = value.cpu().double()
    assert flags.tolist() == [int(f) for f in g["flag"]], (flags.tolist(), g["flag"].tolist())
    W, b = w.module.params["W0"].double(), w.module.params["b0"].double()
    worst = 0.0
    for k in range(N):
        n, s = int(g["neuron"][k]), int(g["sign"][k])
        one = torch.zeros(1, 16, 16, 16, dtype=torch.float64)
        one.view(-1)[n] = 1.0
        row = torch.nn.functional.conv_transpose2d(one, W, stride=2, padding=1).reshape(-1)
        vmax = s * (float(row @ w.spec.center[int(ex[k])].double().reshape(-1)) + float(b[n // 256])) \
            + eps * float(row.abs().sum())
        worst = max(worst, abs(float(value[k]) - vmax))
        assert abs(float(value[k]) - vmax) <= 1e-5 * abs(vmax) + 1e-5, (k, float(value[k]), vmax)
        if int(g["flag"][k]):
            ref = float(g["max_value"][k])
            assert abs(float(value[k]) - ref) <= 1e-5 * abs(ref) + 1e-5, (k, float(value[k]), ref)
    announce(f"  closed {int(flags.sum())}/{N} (reference {int(g['flag'].sum())}), max |value - fp64| {worst:.2e}")


def test_conv_first_layer_two_or_more_splits_match_oracle_and_lp():
    """Two to four split neurons on a conv first layer (where the reference's stacking
    of conv rows cannot broadcast): the device verdicts equal the oracle's, and every
    node the device closes has no point in the box (exact LP on the conv's Jacobian)."""
    from tests.test_oracle_certificate import _conv_lp_trials, _lp_feasible, conv_jacobian
    dev = device()
    announce("split certificate, conv first layer, 2-4 splits per node, vs oracle and LP")
    got, ref = [], []
    for trial, W, b, m, spec, sp, split in _conv_lp_trials(31, 80):
        ref.append(int(ab.split_certificate(m, spec, sp)[0]))
        sd = InputSpec.linf(value_name="input", center=spec.center.to(dev), eps=1.0)
        oshape = tuple(sp["h1"].shape[1:])
        flag = int(split_certificate(_to(m, dev), sd, {"h1": sp["h1"].to(dev)}, {"h1": oshape}).cpu()[0])
        got.append(flag)
        if flag:
            J, off = conv_jacobian(W, b, (1, 3, 3))
            rows = split[0].nonzero().flatten()
            assert not _lp_feasible(J[rows].numpy(), off[rows].numpy(), [-1.0] * 9, [1.0] * 9), trial
    announce(f"  infeasible: hip {sum(got)}, oracle {sum(ref)} of {len(got)}")
    assert sum(ref) >= 3
    assert got == ref


def test_cifar_sized_input_matches_oracle():
    """A 3072-input first layer (3x32x32 flattened: a 12 KB LDS stage of the combined
    normal plus the per-node state): 16 nodes, each splitting a pair of neurons that share
    a weight row and differ in bias by delta in [0.05, 0.15] (both ambiguous: the box's
    radius term is about 0.44), plus two random neurons.  Active on the lower-bias neuron
    and inactive on the other is empty (w.x + b >= 0 and w.x + b + delta <= 0), which the
    Adam search closes with a maximum near -delta / 2 scaled by the pair's weight; the
    reverse is a feasible band.  The device's verdicts and closing maxima equal the
    oracle's, and both verdicts occur."""
    dev = device()
    announce("split certificate vs oracle, 3072 inputs, 16 nodes")
    g = torch.Generator().manual_seed(30)
    I, H = 3072, 64
    x0 = torch.rand(1, I, generator=g)
    eps = 0.01
    W = torch.randn(H // 2, I, generator=g) / I ** 0.5
    W = torch.cat([W, W])
    b0 = -(W[: H // 2] @ x0[0]) + 0.002 * torch.randn(H // 2, generator=g)
    delta = 0.05 + 0.1 * torch.rand(H // 2, generator=g)
    b = torch.cat([b0, b0 + delta])
    m = first_layer_module(W, b)
    nodes = 16
    rows = torch.zeros(nodes, H, dtype=torch.int8)
    for r in range(nodes):
        j = int(torch.randint(0, H // 2, (1,), generator=g))
        rows[r, j], rows[r, j + H // 2] = (1, -1) if r % 2 == 0 else (-1, 1)
        others = [k for k in torch.randperm(H, generator=g).tolist() if k % (H // 2) != j][:2]
        for k in others:
            rows[r, k] = 1 if int(torch.randint(0, 2, (1,), generator=g)) else -1
    ref_flags, ref_vals = [], []
    spec1 = InputSpec.linf(value_name="input", center=x0, eps=eps)
    for r in range(nodes):
        flag, _reason, val = ab.split_certificate(m, spec1, {"h1": rows[r:r + 1]}, return_value=True)
        ref_flags.append(int(flag))
        ref_vals.append(val)
    sd = InputSpec.linf(value_name="input", center=x0.expand(nodes, I).contiguous().to(dev), eps=eps)
    value = torch.empty(nodes, device=dev)
    got = split_certificate(_to(m, dev), sd, {"h1": rows.to(dev)}, {"h1": (H,)}, max_out=value).cpu().tolist()
    announce(f"  infeasible: hip {sum(got)}, oracle {sum(ref_flags)} of {nodes}")
    assert got == ref_flags
    assert 0 < sum(ref_flags) < nodes
    for r in range(nodes):
        if ref_flags[r]:
            v, ref = float(value[r]), float(ref_vals[r])
            assert abs(v - ref) <= 1e-4 * abs(ref) + 1e-6, (r, v, ref)
