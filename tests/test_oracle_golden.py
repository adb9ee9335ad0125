"""Pin the CPU oracle against vectors written by the reference implementation.

The fixtures under tests/golden/ were produced by tests/golden/make_golden.py,
which imports the reference's own runtime (boundflow.runtime.crown_ibp,
alpha_beta_crown, alpha_crown, fused_crown) on the same seeded inputs.  The
oracle restates the same torch operations in the same order, so on the same
torch build the results must agree bit for bit; a tiny tolerance is allowed
only for BLAS threading differences.
"""

import numpy as np
import pytest
import torch

from boundflow_amd import workloads as wl
from oracle import alpha_beta_ref as ab
from oracle import crown_ref as cr
from tests.golden_util import c3_box, dag_case, load, t, workload_checksum


def _close(a, b, rtol=1e-6, atol=1e-6):
    a = torch.as_tensor(a).double()
    b = torch.as_tensor(b).double()
    assert a.shape == b.shape
    assert torch.allclose(a, b, rtol=rtol, atol=atol, equal_nan=True), float((a - b).abs().nan_to_num(0).max())


@pytest.mark.parametrize("tag,maker", [
    ("crown_c1", lambda: wl.make_c1()),
    ("crown_c1_mixed", lambda: wl.make_c1(eps=0.001, label_mode="predicted")),
    ("crown_c3_b16", lambda: wl.subset(wl.make_c3(), 16)),
    ("crown_c3_box", c3_box),
] + [
    (f"crown_dag_{k}{'_box' if b else ''}", (lambda k, b: lambda: dag_case(k, b))(k, b))
    for k in wl.DAG_KINDS for b in (False, True)
])
def test_crown_matches_reference(tag, maker):
    g = load(tag)
    w = maker()
    assert workload_checksum(w) == str(g["checksum"]), "workload generator drifted from the fixture"
    with torch.inference_mode():
        b = cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C)
        _env, pre = cr.forward_ibp_trace(w.module, w.spec)
    _close(b.lower, g["lower"])
    _close(b.upper, g["upper"])
    for i, st in enumerate(pre.values()):
        n = g[f"pre{i}_lower"].shape[0]
        _close(st.lower[:n], g[f"pre{i}_lower"])
        _close(st.upper[:n], g[f"pre{i}_upper"])


def test_all_intermediate_matches_reference_composition():
    g = load("crown_c2_allint_b4")
    w = wl.subset(wl.make_c2(), 4)
    assert workload_checksum(w) == str(g["checksum"])
    with torch.inference_mode():
        final, pre = cr.run_crown_all_intermediate(w.module, w.spec, linear_spec_C=w.C)
    _close(final.lower, g["lower"], rtol=1e-5, atol=1e-5)
    _close(final.upper, g["upper"], rtol=1e-5, atol=1e-5)
    for i, st in enumerate(pre.values()):
        _close(st.lower, g[f"pre{i}_lower"], rtol=1e-5, atol=1e-5)
        _close(st.upper, g[f"pre{i}_upper"], rtol=1e-5, atol=1e-5)


def test_alpha_crown_cnn_matches_reference():
    g = load("alpha_c4_b4")
    w = wl.subset(wl.make_c4(), 4)
    assert workload_checksum(w) == str(g["checksum"])
    _env, pre = cr.forward_ibp_trace(w.module, w.spec)
    init = ab.adaptive_alpha_init(pre)
    for i, a in enumerate(init.values()):
        assert torch.equal(a, t(g[f"init{i}"]))
    bounds, alpha, _beta, _ch = ab.run_alpha_beta_crown(
        w.module, w.spec, linear_spec_C=w.C, steps=20, lr=0.1, warm_start_alpha=init, per_batch_params=True)
    _close(bounds.lower, g["lower"], rtol=1e-5, atol=1e-5)
    _close(bounds.upper, g["upper"], rtol=1e-5, atol=1e-5)
    for i, a in enumerate(alpha.values()):
        _close(a, g[f"alpha{i}"], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("tag,maker", [
    ("bab_c5_d256", lambda: wl.subset(wl.make_c5(), 256)),
    ("bab_c5d2_mixed", lambda: wl.subset(wl.make_c5(eps=0.004, depth=2, label_mode="predicted"), 256)),
])
def test_bab_domain_batch_matches_reference(tag, maker):
    g = load(tag)
    w = maker()
    assert workload_checksum(w) == str(g["checksum"])
    r = ab.evaluate_domain_batch(w.module, w.spec, linear_spec_C=w.C, relu_split_state=w.extra["splits"],
                                 steps=int(w.extra["steps"]), lr=float(w.extra["lr"]))
    assert torch.equal(r["feasible"], t(g["feasible"]))
    assert torch.equal(r["certified"], t(g["certified"]))
    names = list(w.extra["splits"].keys())
    layer = np.array([-1 if b is None else names.index(b[0]) for b in r["branch"]])
    neuron = np.array([-1 if b is None else b[1] for b in r["branch"]])
    assert np.array_equal(layer, g["branch_layer"]) and np.array_equal(neuron, g["branch_neuron"])
    _close(r["lower"], g["lower"], rtol=1e-5, atol=1e-5)
    _close(r["upper"], g["upper"], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("kind", ["linear", "conv2d"])
def test_fused_region_matches_reference(kind):
    g = load(f"fused_{kind}")
    au, bu, al, bl = cr.relu_relax(t(g["l"]), t(g["u"]))
    for x, k in ((au, "alpha_u"), (bu, "beta_u"), (al, "alpha_l"), (bl, "beta_l")):
        assert torch.equal(x, t(g[k]))
    kw = {}
    if kind == "conv2d":
        kw = dict(input_shape=(3, 8, 8), output_shape=(4, 4, 4),
                  attrs={"stride": (2, 2), "padding": (1, 1), "output_padding": (0, 0)})
    out = cr.fused_relu_affine_reference(t(g["A_u"]), t(g["A_l"]), au, al, bu, bl, t(g["weight"]), t(g["bias"]),
                                         kind=kind, **kw)
    for x, k in zip(out, ("A_prev_u", "A_prev_l", "bias_delta_u", "bias_delta_l")):
        _close(x, g[k])


def test_shared_alpha_crown_matches_reference():
    g = load("alpha_shared_mlp")
    gen = torch.Generator().manual_seed(5)
    m = wl.build_mlp([20, 16, 16, 5], gen=gen, bias_std=0.1)
    x = torch.rand(6, 20, generator=gen)
    labels = torch.randint(0, 5, (6,), generator=gen)
    C = wl.margin_spec(labels, 5)
    from boundflow_amd.spec import InputSpec
    spec = InputSpec.linf(value_name="input", center=x, eps=0.1)
    assert workload_checksum(wl.Workload("s", m, spec, C, labels)) == str(g["checksum"])
    bounds, alpha = ab.run_alpha_crown(m, spec, linear_spec_C=C, steps=8, lr=0.2)
    _close(bounds.lower, g["lower"], rtol=1e-5, atol=1e-5)
    _close(bounds.upper, g["upper"], rtol=1e-5, atol=1e-5)
    for i, a in enumerate(alpha.values()):
        _close(a, g[f"alpha{i}"], rtol=1e-4, atol=1e-4)
