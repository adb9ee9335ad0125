"""Conv layers whose maps exceed a 64 KB LDS row stage (16 384 floats): a CNN whose
first conv writes a 32x32x32 map (workloads.make_wide_cnn).  The transposed
convolution of that layer's coefficients and the IBP / gradient convolutions that
read the map take the row kernels' global-memory variant.  Checked against the
oracle (conv_transpose2d / conv2d of torch on the CPU, Conv2dLinearOperator.to_dense,
linear_operator.py:1067-1092, and IntervalDomain.affine_transformer,
domains/interval.py:57-74): IBP pre-activation boxes, CROWN bounds at the contract,
the alpha / beta gradient pass, and the drop-in executor on the wide region."""

import pytest
import torch

from boundflow_amd import alpha_beta as hab
from boundflow_amd import crown as hc
from boundflow_amd import fused_crown as fc
from boundflow_amd import workloads as wl
from oracle import crown_ref as cr
from oracle import parity
from oracle.gradients import oracle_grads, sign_tie_allowances
from tests.gpu_util import announce, assert_bounds_close, assert_parity, assert_verdicts, device

pytestmark = pytest.mark.gpu


def test_wide_cnn_ibp_and_crown_match_oracle():
    dev = device()
    announce("CNN with a 32x32x32 conv map (128 KB per row): IBP and CROWN, B=4")
    w = wl.make_wide_cnn()
    wd = wl.to_device(w, dev)
    trace = hc.forward_ibp_trace(wd.module, wd.spec)
    _env, pre = cr.forward_ibp_trace(w.module, w.spec)
    for name, st in pre.items():
        assert_bounds_close(trace.relu_pre[name].lower, st.lower, f"relu_pre[{name}].lower", atol=1e-5)
        assert_bounds_close(trace.relu_pre[name].upper, st.upper, f"relu_pre[{name}].upper", atol=1e-5)
    got = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
    ref = cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C)
    w64 = parity.to_float64(w)
    ref64 = cr.run_crown_ibp(w64.module, w64.spec, linear_spec_C=w64.C)
    assert_parity(got.lower, ref.lower, ref64.lower, "wide CNN lower")
    assert_parity(got.upper, ref.upper, ref64.upper, "wide CNN upper")
    assert_verdicts(got.lower, ref.lower, ref64.lower, "wide CNN")


def test_wide_cnn_gradients_match_autograd():
    dev = device()
    announce("CNN with a 32x32x32 conv map: dL/dalpha of the lower bound vs autograd")
    w = wl.make_wide_cnn(batch=2)
    g = torch.Generator().manual_seed(8)
    _env, pre = cr.forward_ibp_trace(w.module, w.spec)
    alpha = {k: torch.rand(v.lower.shape, generator=g) for k, v in pre.items()}
    ref32, ga32, _ = oracle_grads(w, alpha)
    ref64, ga64, _ = oracle_grads(w, alpha, dtype=torch.float64)
    wd = wl.to_device(w, dev)
    bounds, ga, _gb = hab.lower_bound_gradients(wd.module, wd.spec, linear_spec_C=wd.C,
                                                relu_alpha={k: v.to(dev) for k, v in alpha.items()})
    assert_parity(bounds.lower, ref32.lower, ref64.lower, "wide CNN lower at alpha")
    allow, _allow_b, nties = sign_tie_allowances(parity.to_float64(w), {k: v.double() for k, v in alpha.items()},
                                                 True)
    announce(f"  {nties} input-layer coefficients within fp32 rounding of zero")
    for k in ga32:
        gh = ga[k].detach().cpu().double().reshape(ga32[k].shape)
        e = ga64[k].double()
        scale = float(e.abs().max()) + 1e-30
        base = max(4.0 * float((ga32[k].double() - e).abs().max()), 1e-5 * scale)
        err = (gh - e).abs()
        announce(f"  dL/dalpha[{k}]: max|hip-fp64| {float(err.max()):.3e}, bound {base:.3e} + allowance")
        assert bool((err <= base + allow[k].double().reshape(err.shape)).all()), k


def test_executor_on_the_wide_region():
    """HipFusedCrownExecutor.run on the ReLU -> conv region of the wide layer (the
    region whose coefficient map is 32x32x32): equal to the oracle's fused region
    (TorchDenseFusedCrownReference.run, fused_crown.py:330-400)."""
    dev = device()
    announce("executor region with a 32x32x32 coefficient map")
    w = wl.make_wide_cnn(batch=2)
    g = torch.Generator().manual_seed(9)
    B, S, n = 2, 9, 32 * 32 * 32
    A_u = torch.randn(B, S, n, generator=g)
    A_l = torch.randn(B, S, n, generator=g)
    au = torch.rand(B, n, generator=g) * 0.9 + 0.1
    bu = torch.rand(B, n, generator=g) * 0.5
    al = (torch.rand(B, n, generator=g) > 0.5).float()
    bl = torch.zeros(B, n)
    W, b = w.module.params["W0"], w.module.params["b0"]
    attrs = {"stride": 1, "padding": 1, "dilation": 1, "groups": 1}
    req = fc.FusedReluAffineRequest(kind="conv2d", A_u=A_u.to(dev), A_l=A_l.to(dev), alpha_u=au.to(dev),
                                    alpha_l=al.to(dev), beta_u=bu.to(dev), beta_l=bl.to(dev), weight=W.to(dev),
                                    bias=b.to(dev), input_shape=(3, 32, 32), output_shape=(32, 32, 32), attrs=attrs)
    ex = fc.HipFusedCrownExecutor()
    ctx = fc.FusedCrownExecutionContext()
    assert ex.supports(req, ctx)
    out = ex.run(req)
    ref = cr.fused_relu_affine_reference(A_u, A_l, au, al, bu, bl, W, b, "conv2d", (3, 32, 32), (32, 32, 32), attrs)
    for name, r in zip(("A_prev_u", "A_prev_l", "bias_delta_u", "bias_delta_l"), ref):
        g64 = getattr(out, name).detach().cpu().double()
        tol = 1e-5 * r.double().abs().max() + 1e-6
        d = float((g64 - r.double()).abs().max())
        announce(f"  {name}: max |hip - ref| {d:.3e} (tol {float(tol):.3e})")
        assert d <= float(tol), name
