"""HIP parity of the drop-in executors: HipTaskExecutor (IBP over BoundTasks)
and HipFusedCrownExecutor (one fused ReLU->affine CROWN region), against the
reference-generated fixtures and the CPU oracle.

Interval affine maps run in center/radius form on the device, where the
reference splits W into W+ and W-; both are exact up to fp32 rounding of the
summed terms, so bounds are compared at rtol 1e-5 with an absolute floor of
1e-5 (intermediate-box tolerance of the IBP forward).
"""

import pytest
import torch

from boundflow_amd import fused_crown as fc
from boundflow_amd import task_executor as te
from boundflow_amd import workloads as wl
from oracle import task_ibp_ref as ti
from tests.golden_util import load, t
from tests.gpu_util import announce, assert_bounds_close, device

pytestmark = pytest.mark.gpu

IBP_CASES = [
    ("task_ibp_c1_b8", lambda: wl.subset(wl.make_c1(), 8)),
    ("task_ibp_c3_b4", lambda: wl.subset(wl.make_c3(), 4)),
    ("task_ibp_dag", lambda: wl.make_ibp_dag()),
    ("task_ibp_dag_box", lambda: wl.make_ibp_dag(box=True)),
]


@pytest.mark.parametrize("tag,maker", IBP_CASES)
def test_task_executor_run_ibp_matches_reference(tag, maker):
    dev = device()
    announce(f"HipTaskExecutor.run_ibp {tag}")
    g = load(tag)
    wd = wl.to_device(maker(), dev)
    out = te.HipTaskExecutor().run_ibp(wd.module, wd.spec)
    torch.cuda.synchronize()
    assert_bounds_close(out.lower, t(g["lower"]), f"{tag} lower", atol=1e-5)
    assert_bounds_close(out.upper, t(g["upper"]), f"{tag} upper", atol=1e-5)


def test_task_executor_scheduled_with_buffer_reuse_matches_reference():
    dev = device()
    announce("run_ibp_scheduled over the three-task DAG split (aliased physical buffers)")
    g = load("task_ibp_dag_sched")
    w = wl.make_ibp_dag()
    mod = wl.split_ibp_dag(wl.to_device(w, dev))
    spec = w.spec.to(dev)
    out = te.run_ibp_scheduled(mod, spec)
    torch.cuda.synchronize()
    assert_bounds_close(out.lower, t(g["lower"]), "scheduled lower", atol=1e-5)
    assert_bounds_close(out.upper, t(g["upper"]), "scheduled upper", atol=1e-5)


@pytest.mark.parametrize("name", ["C2", "C3"])
def test_task_executor_full_size_matches_oracle(name):
    """Full benchmark batch (C2: 256 x 784-500x6-10; C3: 128 x CNN)."""
    dev = device()
    announce(f"HipTaskExecutor.run_ibp full-size {name}")
    w = wl.make(name)
    ref = ti.run_ibp(w.module, w.spec)
    wd = wl.to_device(w, dev)
    out = te.HipTaskExecutor().run_ibp(wd.module, wd.spec)
    torch.cuda.synchronize()
    # deep IBP boxes grow to O(1e2..1e4); compare relative to the box width
    scale = (ref.upper - ref.lower).abs().double().amax(dim=1, keepdim=True).clamp_min(1.0)
    for got, r, what in ((out.lower, ref.lower, "lower"), (out.upper, ref.upper, "upper")):
        err = ((got.cpu().double() - r.double()).abs() / scale).max()
        announce(f"{name} {what}: max error relative to box width {float(err):.3e}")
        assert float(err) <= 1e-5


def _request(tag, kind, dev):
    g = load(tag)
    tt = {k: t(v).to(dev).contiguous() for k, v in g.items()}
    if kind == "linear":
        N, P = tt["weight"].shape
        in_shape, out_shape, attrs = (int(P),), (int(N),), {}
    else:
        in_shape, out_shape = (3, 8, 8), (4, 4, 4)
        attrs = {"stride": (2, 2), "padding": (1, 1), "dilation": (1, 1), "groups": 1, "output_padding": (0, 0)}
    req = fc.FusedReluAffineRequest(kind=kind, A_u=tt["A_u"], A_l=tt["A_l"], alpha_u=tt["alpha_u"],
                                    alpha_l=tt["alpha_l"], beta_u=tt["beta_u"], beta_l=tt["beta_l"],
                                    weight=tt["weight"], bias=tt["bias"], input_shape=in_shape,
                                    output_shape=out_shape, attrs=attrs)
    return req, g


@pytest.mark.parametrize("tag,kind", [("fused_linear", "linear"), ("fused_conv2d", "conv2d")])
def test_hip_fused_crown_executor_matches_reference(tag, kind):
    dev = device()
    announce(f"HipFusedCrownExecutor.run {tag}")
    req, g = _request(tag, kind, dev)
    ex = fc.HipFusedCrownExecutor()
    ctx = fc.FusedCrownExecutionContext()
    assert ex.supports(req, ctx)
    assert not ex.supports(req, fc.FusedCrownExecutionContext(alpha_enabled=True))
    res = ex.run(req)
    torch.cuda.synchronize()
    for k in ("A_prev_u", "A_prev_l", "bias_delta_u", "bias_delta_l"):
        assert_bounds_close(getattr(res, k), t(g[k]), f"{tag} {k}", rtol=1e-5, atol=1e-5)


def test_hip_fused_crown_executor_on_side_stream():
    dev = device()
    announce("HipFusedCrownExecutor.run on a non-default stream")
    req, g = _request("fused_linear", "linear", dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        res = fc.HipFusedCrownExecutor().run(req, stream=s)
    s.synchronize()
    assert_bounds_close(res.A_prev_l, t(g["A_prev_l"]), "side-stream A_prev_l", rtol=1e-5, atol=1e-5)


class _FixtureSession:
    """Stand-in for the reference's Bound IR session (bound_ir_interpreter.py:617-700):
    it assembles the fused region's request from its state (here a reference
    fixture) and runs it through the executor the registry hands it."""

    def __init__(self, tag, kind, dev):
        self.tag, self.kind, self.dev = tag, kind, dev
        self.ran = []

    def execute_fused_relu_affine_task(self, op_ids, *, output_value_ids, executor):
        req, _g = _request(self.tag, self.kind, self.dev)
        if not executor.supports(req, fc.FusedCrownExecutionContext()):
            raise ValueError("executor rejects the region")
        self.ran.append((tuple(op_ids), tuple(output_value_ids)))
        return executor.run(req)


@pytest.mark.parametrize("tag,kind,affine", [("fused_linear", "linear", "linear_backward"),
                                             ("fused_conv2d", "conv2d", "conv2d_backward")])
def test_registry_dispatch_runs_the_hip_kernels(tag, kind, affine):
    """HipTaskBackendRegistry.dispatch (task_backend_dispatch.py:420-533 counterpart)
    drives the HIP executor on a reference fixture: the typed dispatch checks pass,
    the prepared task is cached by the key's hash (a second dispatch hits), and the
    region's bounds equal the reference's."""
    from types import SimpleNamespace as NS
    dev = device()
    announce(f"registry dispatch through HipFusedCrownExecutor: {tag}")
    task = NS(task_id="t0", op_refs=[NS(op_id="relu0", kind=NS(value="relu_relaxation")),
                                     NS(op_id="aff0", kind=NS(value=affine))], output_value_ids=("v_out",))
    template = NS(backend_candidates=[NS(candidate_id="c0", backend=NS(value="hip_fused"), capability_id="cap0")])
    key = NS(backend_candidate_id="c0", stable_hash=lambda: f"key-{tag}")
    reg = fc.HipTaskBackendRegistry()
    sess = _FixtureSession(tag, kind, dev)
    g = load(tag)
    for round_ in range(2):
        res = reg.dispatch(task, key, session=sess, template=template)
        torch.cuda.synchronize()
        for k in ("A_prev_u", "A_prev_l", "bias_delta_u", "bias_delta_l"):
            assert_bounds_close(getattr(res, k), t(g[k]), f"{tag} dispatch {round_} {k}", rtol=1e-5, atol=1e-5)
    assert sess.ran == [(("relu0", "aff0"), ("v_out",))] * 2
    assert (reg.cache_misses, reg.cache_hits) == (1, 1)


@pytest.mark.parametrize("layer", [0, 1])
def test_hip_fused_crown_executor_on_c3_conv_regions(layer):
    """The ReLU -> conv regions of the C3 network (16 channels 16x16 over 3x32x32, and
    32 channels 8x8 over 16x16x16), which the executor runs in one launch (the
    relaxation's four tensors read while the channel-last transposed convolution stages
    each row), against the oracle's fused region (fused_crown.py:330-400), B=4, S=9,
    with synthetic relaxations (both slopes and intercepts nonzero)."""
    from boundflow_amd import workloads as wl
    from oracle import crown_ref as cr
    dev = device()
    announce(f"HipFusedCrownExecutor.run on C3 conv region {layer}")
    w = wl.make_c3()
    W, b = w.module.params[f"W{layer}"], w.module.params[f"b{layer}"]
    in_shape, out_shape = ((3, 32, 32), (16, 16, 16)) if layer == 0 else ((16, 16, 16), (32, 8, 8))
    g = torch.Generator().manual_seed(40 + layer)
    B, S = 4, 9
    n = out_shape[0] * out_shape[1] * out_shape[2]
    A_u, A_l = torch.randn(B, S, n, generator=g), torch.randn(B, S, n, generator=g)
    au = torch.rand(B, n, generator=g) * 0.9 + 0.1
    bu = torch.rand(B, n, generator=g) * 0.5
    al = torch.rand(B, n, generator=g)
    bl = -torch.rand(B, n, generator=g) * 0.1
    b = b + torch.randn(b.shape, generator=g) * 0.1
    attrs = {"stride": 2, "padding": 1, "dilation": 1, "groups": 1}
    req = fc.FusedReluAffineRequest(kind="conv2d", A_u=A_u.to(dev), A_l=A_l.to(dev), alpha_u=au.to(dev),
                                    alpha_l=al.to(dev), beta_u=bu.to(dev), beta_l=bl.to(dev), weight=W.to(dev),
                                    bias=b.to(dev), input_shape=in_shape, output_shape=out_shape, attrs=attrs)
    ex = fc.HipFusedCrownExecutor()
    assert ex.supports(req, fc.FusedCrownExecutionContext())
    res = ex.run(req)
    torch.cuda.synchronize()
    ref = cr.fused_relu_affine_reference(A_u.double(), A_l.double(), au.double(), al.double(), bu.double(),
                                         bl.double(), W.double(), b.double(), "conv2d", in_shape, out_shape, attrs)
    for k, r in zip(("A_prev_u", "A_prev_l", "bias_delta_u", "bias_delta_l"), ref):
        got = getattr(res, k).detach().cpu().double()
        tol = 1e-5 * float(r.abs().max()) + 1e-6
        d = float((got - r).abs().max())
        announce(f"  {k}: max |hip - fp64| {d:.3e} (tol {tol:.3e})")
        assert d <= tol, k
