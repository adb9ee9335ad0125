"""HIP parity of two smaller pieces of the path:

* ``bf_alpha_from_crown`` (the adaptive "from CROWN" slope init,
  native_alpha_beta_optimizer_schedule.py:635-653) at full-size C4: bit-equal to the
  oracle's ``adaptive_alpha_init`` on the same pre-activation boxes, and to the
  reference's init on the first four inputs (fixture alpha_c4_b4, ``init{i}``);
* ``relu_pre_add_coeff_u`` (crown_ibp.py:1270-1278): a term added to the upper
  coefficient after the relaxation, on rank-2 pre-activations (chain MLP and DAG
  networks) against the oracle at the contract, and refused on a conv ReLU with the
  reference's NotImplementedError (:1256-1260)."""

import pytest
import torch

from boundflow_amd import _lib
from boundflow_amd import alpha_beta as hab
from boundflow_amd import crown as hc
from boundflow_amd import workloads as wl
from oracle import alpha_beta_ref as ab
from oracle import crown_ref as cr
from oracle import parity
from tests.golden_util import load, t, workload_checksum
from tests.gpu_util import announce, assert_parity, device

pytestmark = pytest.mark.gpu


def test_alpha_from_crown_full_size_c4():
    dev = device()
    announce("bf_alpha_from_crown at full-size C4 (B=32)")
    w = wl.make_c4()
    _e, pre = cr.forward_ibp_trace(w.module, w.spec)
    ref = ab.adaptive_alpha_init(pre)
    stream = _lib.stream_handle()
    # on the oracle's own boxes: bit-equal
    for name, st in pre.items():
        lo, hi = st.lower.to(dev).contiguous(), st.upper.to(dev).contiguous()
        a = torch.empty_like(lo)
        _lib.call("bf_alpha_from_crown", _lib.ptr(lo), _lib.ptr(hi), lo.numel(), _lib.ptr(a), stream)
        assert torch.equal(a.cpu(), ref[name]), name
    # on the device's boxes: the init the HIP optimiser starts from
    wd = wl.to_device(w, dev)
    trace = hc.forward_ibp_trace(wd.module, wd.spec)
    got = hab.alpha_from_crown(trace)
    g = load("alpha_c4_b4")
    assert workload_checksum(wl.subset(w, 4)) == str(g["checksum"])
    for i, name in enumerate(pre):
        h = got[name].cpu()
        lo, hi = pre[name].lower, pre[name].upper
        # a neuron whose u + l is within the two fp32 boxes' difference may flip the adaptive choice
        tie = (hi + lo).abs() <= (trace.relu_pre[name].upper.cpu() - hi).abs() + (trace.relu_pre[name].lower.cpu()
                                                                                  - lo).abs()
        diff = h != ref[name]
        announce(f"  {name}: {int(diff.sum())}/{h.numel()} differ from the oracle's init, all at ties: "
                 f"{bool((~diff | tie).all())}")
        assert bool((~diff | tie).all()), name
        assert torch.equal(h[:4], t(g[f"init{i}"])), f"{name} vs the reference's init"


@pytest.mark.parametrize("kind", ["mlp", "dag"])
def test_upper_split_term_matches_oracle(kind):
    dev = device()
    announce(f"relu_pre_add_coeff_u on a {kind}")
    gen = torch.Generator().manual_seed(23)
    if kind == "mlp":
        w = wl.subset(wl.make_c1(eps=0.01), 8)
    else:
        w = wl.make_dag("residual_mlp", batch=6)
    _e, pre = cr.forward_ibp_trace(w.module, w.spec)
    add_u = {k: torch.randn(v.lower.shape, generator=gen) * 0.05 for k, v in pre.items()}
    add_l = {k: -torch.rand(v.lower.shape, generator=gen) * 0.05 for k, v in pre.items()}
    kw = dict(linear_spec_C=w.C, relu_pre_add_coeff_u=add_u, relu_pre_add_coeff_l=add_l)
    ref = cr.run_crown_ibp(w.module, w.spec, **kw)
    w64 = parity.to_float64(w)
    ref64 = cr.run_crown_ibp(w64.module, w64.spec, linear_spec_C=w64.C,
                             relu_pre_add_coeff_u={k: v.double() for k, v in add_u.items()},
                             relu_pre_add_coeff_l={k: v.double() for k, v in add_l.items()})
    wd = wl.to_device(w, dev)
    got = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C,
                               relu_pre_add_coeff_u={k: v.to(dev) for k, v in add_u.items()},
                               relu_pre_add_coeff_l={k: v.to(dev) for k, v in add_l.items()})
    assert_parity(got.lower, ref.lower, ref64.lower, f"{kind} lower with split terms")
    assert_parity(got.upper, ref.upper, ref64.upper, f"{kind} upper with split terms")
    # the term moves the upper bound: without it the bounds differ
    plain = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C,
                                 relu_pre_add_coeff_l={k: v.to(dev) for k, v in add_l.items()})
    assert not torch.equal(plain.upper, got.upper)


def test_upper_split_term_refused_on_conv_relu():
    dev = device()
    announce("relu_pre_add_coeff_u on a conv ReLU")
    w = wl.subset(wl.make_c3(), 2)
    wd = wl.to_device(w, dev)
    add_u = {"h0": torch.zeros(2, 16, 16, 16, device=dev)}
    with pytest.raises(NotImplementedError, match="only supports relu_pre_add_coeff_u on rank-2 pre-activations"):
        hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C, relu_pre_add_coeff_u=add_u)
    with pytest.raises(NotImplementedError, match="only supports relu_pre_add_coeff_u on rank-2 pre-activations"):
        cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C, relu_pre_add_coeff_u={"h0": torch.zeros(2, 16, 16, 16)})
