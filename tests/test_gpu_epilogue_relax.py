"""HIP parity tests of the relaxation fused into the epilogue of the contraction
that produces the coefficient (bf_crown_relu_linear_relu_fwd) and of the
concretization of an already relaxed coefficient (bf_crown_linear_concretize).

The two-region step is checked against the oracle's dense ReLU backward
(oracle/crown_ref.py: relu_backward_dense, crown_ibp.py:1211-1298) composed with
the linear step in float64; whole CROWN queries that take the epilogue path
(>= 15 spec rows per domain) are checked against the oracle's run_crown_ibp with
alpha slopes and beta split coefficients, for Linf and box inputs."""

import pytest
import torch

from boundflow_amd import _lib
from boundflow_amd import crown as hc
from boundflow_amd import workloads as wl
from boundflow_amd.spec import InputSpec
from oracle import crown_ref as cr
from oracle import parity
from tests.gpu_util import announce, assert_bounds_close, assert_parity, assert_verdicts, device

pytestmark = pytest.mark.gpu


def _pre(D, n, g):
    lo = torch.randn(D, n, generator=g)
    hi = lo + torch.rand(D, n, generator=g) * 1.5
    # stably inactive at 0, inactive, active, and zero-width cases in the first columns
    lo[:, :4] = torch.tensor([0.0, -1.0, 0.5, 0.0])
    hi[:, :4] = torch.tensor([0.0, 0.0, 1.0, 2.0])
    return lo, hi


def _table(lo, hi, alpha, dev):
    D, n = lo.shape
    t = torch.empty(D, n, 4, device=dev)
    lo_d, hi_d = lo.to(dev).contiguous(), hi.to(dev).contiguous()
    a_d = None if alpha is None else alpha.to(dev).contiguous()
    _lib.call("bf_relu_relax_table", _lib.ptr(lo_d), _lib.ptr(hi_d), _lib.ptr(a_d), n, D, n, _lib.ptr(t),
              _lib.stream_handle())
    return t, (lo_d, hi_d, a_d)


# S = 20 and 40: a 128-row tile spans <= 10 domains (entries staged in LDS);
# S = 9: up to 16 domains per tile (entries read from global memory).  N <= 16 with no
# prologue relaxation: the short-contraction kernel (a wave per domain and 256 columns;
# P = 300 gives two column chunks, the second partial), with or without the region's bias.
# D = 2048 with the plain prologue: 18 432 rows, a grid that takes the 64 x 128 tile
# configuration (its 128 x 128 tiles would load the CUs unevenly).
@pytest.mark.parametrize("S,prologue,alpha,add,cvec,N,bias_only,D", [
    (20, True, True, True, True, 150, False, 13),
    (20, False, False, False, False, 150, False, 13),
    (9, True, False, True, True, 150, False, 13),
    (40, False, True, True, False, 150, False, 13),
    (9, False, True, True, True, 10, True, 13),
    (20, False, False, False, False, 16, False, 13),
    (3, False, True, False, True, 7, True, 13),
    (9, False, True, True, True, 150, False, 2048),
])
def test_two_region_step_matches_oracle(S, prologue, alpha, add, cvec, N, bias_only, D):
    dev = device()
    announce(f"relax epilogue step D={D} S={S} N={N} prologue={prologue} bias_only={bias_only} alpha={alpha} "
             f"add={add} cvec={cvec}")
    g = torch.Generator().manual_seed(S * 3 + prologue + N)
    P = 300
    if D > 13:
        assert chr(_lib.load().bf_gemm_tile_config(D * S, P, 2, 1, 0, 1)) == "Q"
    A_u = torch.randn(D, S, N, generator=g)
    A_l = torch.randn(D, S, N, generator=g)
    l1, u1 = _pre(D, N, g)
    l2, u2 = _pre(D, P, g)
    a1 = torch.rand(D, N, generator=g) if alpha else None
    a2 = torch.rand(D, P, generator=g) if alpha else None
    add1 = torch.randn(D, N, generator=g) if add else None
    add2 = torch.randn(D, P, generator=g) if add else None
    W = torch.randn(N, P, generator=g) * 0.1          # layer weight [out = N, in = P]
    bias1 = torch.randn(N, generator=g)
    bias2 = torch.randn(P, generator=g)
    cv = torch.randn(D, P, generator=g) if cvec else None
    b_u = torch.randn(D, S, generator=g)
    b_l = torch.randn(D, S, generator=g)

    # oracle, float64: [prologue relaxation + bias] -> A' W -> relaxation of the next ReLU + its bias
    f = lambda x: None if x is None else x.double()
    Au, Al, bu, bl = f(A_u), f(A_l), f(b_u), f(b_l)
    if prologue:
        Au, Al, bu, bl = cr.relu_backward_dense(
            Au, Al, bu, bl, pre=cr.IntervalState(f(l1), f(u1)), name="h1",
            relu_alpha=None if a1 is None else {"h1": f(a1)}, add_l=None if add1 is None else {"h1": f(add1)})
        bu = bu + Au @ f(bias1)
        bl = bl + Al @ f(bias1)
    elif bias_only:
        bu = bu + Au @ f(bias1)
        bl = bl + Al @ f(bias1)
    Cu, Cl = Au @ f(W), Al @ f(W)
    Cu2, Cl2, bu2, bl2 = cr.relu_backward_dense(
        Cu, Cl, bu, bl, pre=cr.IntervalState(f(l2), f(u2)), name="h2",
        relu_alpha=None if a2 is None else {"h2": f(a2)}, add_l=None if add2 is None else {"h2": f(add2)})
    bu2 = bu2 + Cu2 @ f(bias2)
    bl2 = bl2 + Cl2 @ f(bias2)

    # HIP
    d = lambda x: None if x is None else x.to(dev).contiguous()
    t1, keep1 = _table(l1, u1, a1, dev) if prologue else (None, None)
    t2, keep2 = _table(l2, u2, a2, dev)
    Au_d, Al_d, Wt_d = d(A_u), d(A_l), d(W.t())
    add1_d, add2_d, bias1_d, bias2_d, cv_d = d(add1), d(add2), d(bias1), d(bias2), d(cv)
    bu_d, bl_d = d(b_u), d(b_l)
    M = D * S
    ws = torch.empty(int(_lib.load().bf_crown_relu_linear_relu_fwd_workspace(D, S, P)), device=dev)
    An_u, An_l = torch.empty(M, P, device=dev), torch.empty(M, P, device=dev)
    bo_u, bo_l = torch.empty(M, device=dev), torch.empty(M, device=dev)
    co_u = torch.empty(M, device=dev) if cvec else None
    co_l = torch.empty(M, device=dev) if cvec else None
    Pre_u = torch.empty(M, P, device=dev) if alpha else None   # the product before the relaxation (optional)
    Pre_l = torch.empty(M, P, device=dev) if alpha else None
    _lib.call("bf_crown_relu_linear_relu_fwd", _lib.ptr(Au_d), _lib.ptr(Al_d), S * N, D, S, N, _lib.ptr(t1),
              _lib.ptr(add1_d if prologue else None), N, _lib.ptr(Wt_d), P,
              _lib.ptr(bias1_d if prologue or bias_only else None), _lib.ptr(bu_d), _lib.ptr(bl_d), _lib.ptr(t2),
              _lib.ptr(add2_d), P, _lib.ptr(bias2_d), _lib.ptr(cv_d), P, _lib.ptr(ws), _lib.ptr(An_u),
              _lib.ptr(An_l), _lib.ptr(Pre_u), _lib.ptr(Pre_l), _lib.ptr(bo_u), _lib.ptr(bo_l), _lib.ptr(co_u),
              _lib.ptr(co_l), _lib.stream_handle())
    torch.cuda.synchronize()

    # fp32 accumulation bounds: contraction over N (and the prologue's sums), then the row sums over P
    absA = (Au.abs() if prologue else f(A_u).abs())
    tolC = N * 2.0 ** -22 * (absA @ f(W).abs()) + 1e-6
    for got, ref, what in ((An_u, Cu2, "A_next upper"), (An_l, Cl2, "A_next lower")):
        err = (got.cpu().double().reshape(D, S, P) - ref).abs()
        announce(f"  {what}: max abs err {float(err.max()):.3e}")
        assert bool((err <= tolC).all()), f"{what}: {float((err / tolC).max()):.3f} x tolerance"
    scale_u = (Cu.abs() @ torch.ones(P, dtype=torch.float64) * 2 + Cu2.abs() @ f(bias2).abs() + bu.abs()
               + (absA @ f(bias1).abs() if prologue or bias_only else 0) + 1.0)
    scale_l = (Cl.abs() @ torch.ones(P, dtype=torch.float64) * 2 + Cl2.abs() @ f(bias2).abs() + bl.abs()
               + (absA @ f(bias1).abs() if prologue or bias_only else 0) + 1.0)
    for got, ref, sc, what in ((bo_u, bu2, scale_u, "b upper"), (bo_l, bl2, scale_l, "b lower")):
        err = (got.cpu().double().reshape(D, S) - ref).abs()
        tol = (N + P) * 2.0 ** -22 * sc
        announce(f"  {what}: max abs err {float(err.max()):.3e}")
        assert bool((err <= tol).all()), f"{what}: {float((err / tol).max()):.3f} x tolerance"
    if alpha:
        for got, ref, what in ((Pre_u, Cu, "pre-relaxation upper"), (Pre_l, Cl, "pre-relaxation lower")):
            err = (got.cpu().double().reshape(D, S, P) - ref).abs()
            assert bool((err <= tolC).all()), f"{what}: {float((err / tolC).max()):.3f} x tolerance"
    if cvec:
        for got, C2, what in ((co_u, Cu2, "center upper"), (co_l, Cl2, "center lower")):
            ref = (C2 * f(cv)[:, None, :]).sum(-1)
            tol = P * 2.0 ** -22 * ((C2.abs() * f(cv).abs()[:, None, :]).sum(-1) + tolC.sum(-1)) + 1e-6
            err = (got.cpu().double().reshape(D, S) - ref).abs()
            announce(f"  {what}: max abs err {float(err.max()):.3e}")
            assert bool((err <= tol).all()), f"{what}: {float((err / tol).max()):.3f} x tolerance"


def test_plain_fwd_without_relaxation_passes_bias_through():
    """bf_crown_relu_linear_fwd with no table, split term or bias: the plain
    contraction, and b_out equals b_in."""
    dev = device()
    announce("fused fwd without relaxation = plain contraction")
    g = torch.Generator().manual_seed(3)
    D, S, N, P = 7, 11, 90, 140
    A = torch.randn(D * S, N, generator=g)
    W = torch.randn(N, P, generator=g)
    b = torch.randn(D * S, generator=g)
    Ad, Wt, bd = A.to(dev), W.t().contiguous().to(dev), b.to(dev)
    C = torch.empty(D * S, P, device=dev)
    bo = torch.empty(D * S, device=dev)
    _lib.call("bf_crown_relu_linear_fwd", None, _lib.ptr(Ad), S * N, D, S, N, None, None, 0, _lib.ptr(Wt), P, 1,
              None, None, _lib.ptr(bd), None, _lib.ptr(C), None, _lib.ptr(bo), _lib.stream_handle())
    torch.cuda.synchronize()
    ref = A.double() @ W.double()
    tol = N * 2.0 ** -22 * (A.double().abs() @ W.double().abs())
    assert bool(((C.cpu().double() - ref).abs() <= tol).all())
    assert torch.equal(bo.cpu(), b)


def _with_spec(w, spec, C):
    return wl.Workload(w.name, w.module, spec, C, w.labels, {})


@pytest.mark.parametrize("box,shared", [(False, False), (True, False), (False, True)])
def test_crown_query_on_epilogue_path_matches_oracle(box, shared, monkeypatch):
    """A CROWN query with 20 spec rows per domain (the epilogue path at every hidden
    layer), alpha slopes and beta split coefficients on every ReLU.  shared: one
    [20, 10] spec matrix for every domain, whose first relaxation is materialized
    per domain by the relaxation pass before the plain contraction."""
    dev = device()
    monkeypatch.setattr(hc, "EPILOGUE_MIN_M", 0)   # the epilogue path at this small size
    announce(f"CROWN query on the relaxation-epilogue path, box={box} shared={shared}")
    B, S = 12, 20
    w = wl.make_c2(batch=B, width=200, depth=4)
    g = torch.Generator().manual_seed(17)
    C = torch.randn(S, 10, generator=g) if shared else torch.randn(B, S, 10, generator=g)
    x = w.spec.center
    if box:
        spec = InputSpec.box(value_name="input", lower=(x - 0.02).clamp(0, 1), upper=(x + 0.02).clamp(0, 1))
    else:
        spec = InputSpec.linf(value_name="input", center=x, eps=0.01)
    w = _with_spec(w, spec, C)
    names = wl.relu_input_names(w.module)
    alpha = {n: torch.rand(B, 200, generator=g) for n in names}
    add = {n: torch.randn(B, 200, generator=g) * 0.05 for n in names}
    ref = cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C, relu_alpha=alpha, relu_pre_add_coeff_l=add)
    w64 = parity.to_float64(w)
    ref64 = cr.run_crown_ibp(w64.module, w64.spec, linear_spec_C=w64.C,
                             relu_alpha={k: v.double() for k, v in alpha.items()},
                             relu_pre_add_coeff_l={k: v.double() for k, v in add.items()})
    wd = wl.to_device(w, dev)
    b = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C,
                             relu_alpha={k: v.to(dev) for k, v in alpha.items()},
                             relu_pre_add_coeff_l={k: v.to(dev) for k, v in add.items()})
    torch.cuda.synchronize()
    assert_parity(b.lower, ref.lower, ref64.lower, "epilogue path lower")
    assert_parity(b.upper, ref.upper, ref64.upper, "epilogue path upper")
    assert_verdicts(b.lower, ref.lower, ref64.lower, "epilogue path")


def test_multi_table_launch_equals_single_tables():
    """bf_relu_relax_table_multi: each table bit-equal to bf_relu_relax_table's, with and
    without alpha (per-domain and shared rows), an empty table among them, and more
    tables than one launch takes (17, two launches)."""
    dev = device()
    announce("bf_relu_relax_table_multi: 17 tables, D=7")
    g = torch.Generator().manual_seed(41)
    D = 7
    widths = [5, 300, 0, 64, 1] + [33 + 7 * i for i in range(12)]
    lo, hi, al, ld, want, got = [], [], [], [], [], []
    for i, n in enumerate(widths):
        l, h = _pre(D, n, g) if n >= 4 else (torch.randn(D, n, generator=g), torch.randn(D, n, generator=g).abs())
        h = torch.maximum(h, l)
        a = None if i % 3 == 0 else torch.rand(D if i % 3 == 1 else 1, n, generator=g) * 1.4 - 0.2
        lo.append(l.to(dev).contiguous())
        hi.append(h.to(dev).contiguous())
        al.append(None if a is None else a.to(dev).contiguous())
        ld.append(n if i % 3 == 1 else 0)
        w = torch.empty(D, n, 4, device=dev)
        _lib.call("bf_relu_relax_table", _lib.ptr(lo[-1]), _lib.ptr(hi[-1]), _lib.ptr(al[-1]), ld[-1], D, n,
                  _lib.ptr(w), _lib.stream_handle())
        want.append(w)
        got.append(torch.full((D, n, 4), float("nan"), device=dev))
    _lib.call("bf_relu_relax_table_multi", len(widths), _lib.ptr_array(lo), _lib.ptr_array(hi), _lib.ptr_array(al),
              _lib.i64_array(ld), D, _lib.i64_array(widths), _lib.ptr_array(got), _lib.stream_handle())
    torch.cuda.synchronize()
    for i, (w, t) in enumerate(zip(want, got)):
        assert torch.equal(w.cpu(), t.cpu()), f"table {i} (K={widths[i]})"
