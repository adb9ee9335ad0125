"""HIP parity tests for the linear (MLP) CROWN path, checked against the CPU
oracle and the reference-generated golden vectors."""

import pytest
import torch

from boundflow_amd import _lib
from boundflow_amd import crown as hc
from boundflow_amd import workloads as wl
from oracle import alpha_beta_ref as ab
from oracle import crown_ref as cr
from tests.golden_util import load, t
from oracle import parity
from tests.gpu_util import announce, assert_bounds_close, assert_parity, assert_verdicts, contraction_tol, device

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K,trans_b,abs_b", [
    (37, 19, 5, 0, 0), (128, 128, 16, 0, 0), (300, 257, 130, 1, 0), (576, 784, 256, 0, 0),
    (1000, 500, 500, 1, 1), (9, 10, 10, 0, 0),
])
def test_gemm_matches_fp64(M, N, K, trans_b, abs_b):
    dev = device()
    announce(f"gemm M={M} N={N} K={K} trans_b={trans_b} abs_b={abs_b}")
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(M, K, generator=g)
    B = torch.randn(N, K, generator=g) if trans_b else torch.randn(K, N, generator=g)
    Bm = B.t() if trans_b else B
    if abs_b:
        Bm = Bm.abs()
    ref = A.double() @ Bm.double()
    C = torch.empty(M, N, device=dev)
    Ad, Bd = A.to(dev), B.to(dev)
    _lib.call("bf_gemm", _lib.ptr(Ad), K, _lib.ptr(Bd), (K if trans_b else N), trans_b, abs_b, _lib.ptr(C), N,
              M, N, K, _lib.stream_handle())
    torch.cuda.synchronize()
    tol = contraction_tol(A, Bm, K) + 1e-30
    err = (C.cpu().double() - ref).abs()
    assert bool((err <= tol).all()), float((err / tol).max())


@pytest.mark.parametrize("M,N,K,S", [(288, 100, 2048, 9), (2304, 784, 256, 9), (36, 10, 100, 9), (500, 40, 4000, 5)])
def test_gemm_rank1_split_k_matches_fp64(M, N, K, S):
    """bf_gemm_rank1 (gradient contraction g . W^T + r_row x v_col): the split-K
    path (skinny outputs) and the unsplit path against float64, and the split
    result is identical on a second run (chunks are summed in a fixed order)."""
    dev = device()
    announce(f"gemm_rank1 M={M} N={N} K={K} S={S}")
    g = torch.Generator().manual_seed(M + K)
    A = torch.randn(M, K, generator=g)
    W = torch.randn(N, K, generator=g)
    r = torch.randn(M, generator=g)
    D = (M + S - 1) // S
    v = torch.randn(D, N, generator=g)
    ref = A.double() @ W.double().t() + r.double()[:, None] * v.double()[torch.arange(M) // S]
    tol = contraction_tol(A, W.t(), K) + (r.double()[:, None] * v.double()[torch.arange(M) // S]).abs() * 2.0 ** -22
    Ad, Wd, rd, vd = A.to(dev), W.to(dev), r.to(dev), v.to(dev)
    wsz = int(_lib.load().bf_gemm_rank1_workspace(M, N, K))
    ws = torch.empty(max(wsz, 1), device=dev)
    outs = []
    for use_ws in (True, True, False):
        C = torch.empty(M, N, device=dev)
        _lib.call("bf_gemm_rank1", _lib.ptr(Ad), K, _lib.ptr(Wd), K, 1, _lib.ptr(C), N, M, N, K, S, _lib.ptr(rd),
                  _lib.ptr(vd), N, _lib.ptr(ws) if use_ws else None, wsz if use_ws else 0, _lib.stream_handle())
        outs.append(C)
    torch.cuda.synchronize()
    announce(f"  split workspace floats {wsz}")
    for C in outs:
        err = (C.cpu().double() - ref).abs()
        assert bool((err <= tol).all()), float((err / tol).max())
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("w_trans", [0, 1])
def test_fused_relu_linear_region_golden(w_trans):
    dev = device()
    announce(f"fused relu+linear region vs reference fixture (w_trans={w_trans})")
    gz = load("fused_linear")
    A_u, A_l = t(gz["A_u"]), t(gz["A_l"])
    D, S, N = A_u.shape
    W = t(gz["weight"])
    P = int(W.shape[1])
    outs = [torch.empty(D * S, P, device=dev), torch.empty(D * S, P, device=dev),
            torch.empty(D * S, device=dev), torch.empty(D * S, device=dev)]
    args = [x.to(dev).contiguous() for x in (A_u, A_l, t(gz["l"]), t(gz["u"]), W, t(gz["bias"]))]
    table = torch.empty(D, N, 4, device=dev)
    _lib.call("bf_relu_relax_table", _lib.ptr(args[2]), _lib.ptr(args[3]), None, 0, D, N, _lib.ptr(table),
              _lib.stream_handle())
    # the table holds exactly the executor request's alpha_u, beta_u, alpha_l, beta_l
    for i, k in enumerate(("alpha_u", "beta_u", "alpha_l", "beta_l")):
        assert torch.equal(table[..., i].cpu(), t(gz[k])), k
    Wop = args[4].t().contiguous() if w_trans else args[4]
    _lib.call("bf_crown_relu_linear_fwd", _lib.ptr(args[0]), _lib.ptr(args[1]), S * N, D, S, N, _lib.ptr(table),
              None, 0, _lib.ptr(Wop), P, w_trans, _lib.ptr(args[5]), None, None,
              _lib.ptr(outs[0]), _lib.ptr(outs[1]), _lib.ptr(outs[2]), _lib.ptr(outs[3]), _lib.stream_handle())
    torch.cuda.synchronize()
    assert_bounds_close(outs[0].reshape(D, S, P), t(gz["A_prev_u"]), "A_prev_u", rtol=1e-5, atol=1e-5)
    assert_bounds_close(outs[1].reshape(D, S, P), t(gz["A_prev_l"]), "A_prev_l", rtol=1e-5, atol=1e-5)
    assert_bounds_close(outs[2].reshape(D, S), t(gz["bias_delta_u"]), "bias_delta_u", rtol=1e-5, atol=1e-5)
    assert_bounds_close(outs[3].reshape(D, S), t(gz["bias_delta_l"]), "bias_delta_l", rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("tag,maker", [
    ("crown_c1", lambda: wl.make_c1()),
    ("crown_c1_mixed", lambda: wl.make_c1(eps=0.001, label_mode="predicted")),
])
def test_crown_mlp_matches_reference(tag, maker):
    dev = device()
    announce(f"run_crown_ibp_mlp {tag}")
    gz = load(tag)
    w = maker()
    wd = wl.to_device(w, dev)
    trace = hc.forward_ibp_trace(wd.module, wd.spec)
    # Intermediate IBP boxes: the reference sums l.W+ and u.W- separately (cancellation near 0),
    # the HIP path uses the center/radius form; both carry fp32 rounding of the summed terms, so
    # near-zero entries are compared with an absolute floor of 1e-5.
    for i, st in enumerate(trace.relu_pre.values()):
        n = gz[f"pre{i}_lower"].shape[0]
        assert_bounds_close(st.lower[:n], t(gz[f"pre{i}_lower"]), f"{tag} relu_pre[{i}].lower", atol=1e-5)
        assert_bounds_close(st.upper[:n], t(gz[f"pre{i}_upper"]), f"{tag} relu_pre[{i}].upper", atol=1e-5)
    b = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
    torch.cuda.synchronize()
    w64 = parity.to_float64(w)
    ref64 = cr.run_crown_ibp(w64.module, w64.spec, linear_spec_C=w64.C)
    assert_parity(b.lower, t(gz["lower"]), ref64.lower, f"{tag} lower")
    assert_parity(b.upper, t(gz["upper"]), ref64.upper, f"{tag} upper")
    assert_verdicts(b.lower, t(gz["lower"]), ref64.lower, tag)


def test_crown_mlp_with_splits_matches_oracle():
    dev = device()
    announce("run_crown_ibp_mlp with per-domain splits (C5 network, 64 domains)")
    w = wl.subset(wl.make_c5(eps=0.004, depth=2, label_mode="predicted"), 64)
    feas = ab.domain_feasible(w.module, w.spec, w.extra["splits"])
    idx = feas.nonzero().flatten()
    w = wl.Workload(w.name, w.module,
                    type(w.spec)(value_name="input", center=w.spec.center[idx], perturbation=w.spec.perturbation),
                    w.C[idx], w.labels[idx], {"splits": {k: v[idx] for k, v in w.extra["splits"].items()}})
    ref = cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C, relu_split_state=w.extra["splits"])
    w64 = parity.to_float64(w)
    ref64 = cr.run_crown_ibp(w64.module, w64.spec, linear_spec_C=w64.C, relu_split_state=w64.extra["splits"])
    wd = wl.to_device(w, dev)
    b = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C, relu_split_state=wd.extra["splits"])
    assert_parity(b.lower, ref.lower, ref64.lower, "split lower")
    assert_parity(b.upper, ref.upper, ref64.upper, "split upper")
    assert_verdicts(b.lower, ref.lower, ref64.lower, "split")


def test_infeasible_split_raises_and_flags():
    dev = device()
    announce("infeasible split -> ValueError / per-domain flag")
    w = wl.subset(wl.make_c5(), 8)
    wd = wl.to_device(w, dev)
    names = wl.relu_input_names(w.module)
    trace = hc.forward_ibp_trace(wd.module, wd.spec, raise_on_infeasible=False)
    # force domain 3 to split a stably-inactive neuron active
    u = trace.relu_pre[names[0]].upper[3].cpu()
    j = int(torch.argmin(u))
    assert float(u[j]) < 0
    split = {k: v.clone() for k, v in wd.extra["splits"].items()}
    split[names[0]][3, j] = 1
    tr = hc.forward_ibp_trace(wd.module, wd.spec, relu_split_state=split, raise_on_infeasible=False)
    flags = tr.infeasible.cpu()
    assert int(flags[3]) == 1
    with pytest.raises(ValueError):
        hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C, relu_split_state=split)


# epilogue: the regions relaxed in the producing contraction's epilogue, the path of C2
# at full size (at least EPILOGUE_MIN_M rows), taken here at the fixture's size
@pytest.mark.parametrize("epilogue", [False, True])
def test_all_intermediate_c2_matches_reference(epilogue, monkeypatch):
    dev = device()
    if epilogue:
        monkeypatch.setattr(hc, "EPILOGUE_MIN_M", 0)
    announce(f"C2 all-intermediate CROWN, B=4, epilogue={epilogue}")
    gz = load("crown_c2_allint_b4")
    w = wl.subset(wl.make_c2(), 4)
    wd = wl.to_device(w, dev)
    final, pre = hc.run_crown_all_intermediate(wd.module, wd.spec, linear_spec_C=wd.C)
    for i, st in enumerate(pre.values()):
        assert_bounds_close(st.lower, t(gz[f"pre{i}_lower"]), f"C2 pre{i} lower", rtol=1e-5, atol=1e-5)
        assert_bounds_close(st.upper, t(gz[f"pre{i}_upper"]), f"C2 pre{i} upper", rtol=1e-5, atol=1e-5)
    w64 = parity.to_float64(w)
    ref64, _ = cr.run_crown_all_intermediate(w64.module, w64.spec, linear_spec_C=w64.C)
    assert_parity(final.lower, t(gz["lower"]), ref64.lower, "C2 lower")
    assert_parity(final.upper, t(gz["upper"]), ref64.upper, "C2 upper")


@pytest.mark.parametrize("K", [132, 133, 500])
def test_relax_pass_of_shared_coefficient(K):
    """bf_crown_relu_relax with a_dstride = 0: one [S, K] coefficient shared by every
    domain, relaxed per domain into [D*S, K] (the first region of a C = I query)."""
    dev = device()
    announce(f"relax pass of a shared coefficient K={K}")
    g = torch.Generator().manual_seed(K)
    D, S = 6, 17
    A = torch.randn(S, K, generator=g)
    l = torch.randn(D, K, generator=g)
    u = l + torch.rand(D, K, generator=g)
    alpha = torch.rand(D, K, generator=g)
    kb = torch.randn(K, generator=g)
    b = torch.randn(D, S, generator=g)
    Ab = A.expand(D, S, K)
    ref = cr.relu_backward_dense(Ab, Ab, b, b, pre=cr.IntervalState(l, u), name="h", relu_alpha={"h": alpha})
    # bias sums in float64, with the fp32 summation bound K * 2^-22 * sum |terms| as tolerance
    f = lambda x: x.double()
    r64 = cr.relu_backward_dense(f(Ab), f(Ab), f(b), f(b), pre=cr.IntervalState(f(l), f(u)), name="h",
                                 relu_alpha={"h": f(alpha)})
    ref_bu, ref_bl = r64[2] + r64[0] @ f(kb), r64[3] + r64[1] @ f(kb)
    # |beta_sel| <= max(|l|, |u|): bound of the summed terms A * beta_sel and A' * kbias, plus the input bias
    scale = ((f(Ab).abs() * torch.maximum(f(l).abs(), f(u).abs())[:, None, :]).sum(-1)
             + torch.maximum(r64[0].abs(), r64[1].abs()) @ f(kb).abs() + f(b).abs())
    d = [x.to(dev).contiguous() for x in (A, l, u, alpha, kb, b)]
    table = torch.empty(D, K, 4, device=dev)
    _lib.call("bf_relu_relax_table", _lib.ptr(d[1]), _lib.ptr(d[2]), _lib.ptr(d[3]), K, D, K, _lib.ptr(table),
              _lib.stream_handle())
    out = [torch.empty(D * S, K, device=dev), torch.empty(D * S, K, device=dev), torch.empty(D * S, device=dev),
           torch.empty(D * S, device=dev)]
    _lib.call("bf_crown_relu_relax", _lib.ptr(d[0]), _lib.ptr(d[0]), 0, D, S, K, _lib.ptr(table), None, 0,
              _lib.ptr(d[4]), None, _lib.ptr(d[5]), _lib.ptr(d[5]), _lib.ptr(out[0]), _lib.ptr(out[1]),
              _lib.ptr(out[2]), _lib.ptr(out[3]), None, None, _lib.stream_handle())
    torch.cuda.synchronize()
    assert torch.equal(out[0].cpu().reshape(D, S, K), ref[0])
    assert torch.equal(out[1].cpu().reshape(D, S, K), ref[1])
    for got, ref_b, what in ((out[2], ref_bu, "b_u"), (out[3], ref_bl, "b_l")):
        err = (got.cpu().double().reshape(D, S) - ref_b).abs()
        tol = 2 * K * 2.0 ** -23 * scale
        announce(f"  shared relax {what}: max abs err {float(err.max()):.3e}")
        assert bool((err <= tol).all()), f"{what}: {float((err / tol).max()):.3f} x tolerance"


@pytest.mark.parametrize("K,S,same", [(256, 150, True), (500, 150, False), (512, 64, True), (132, 20, False)])
def test_shared_coefficient_pass_equals_per_domain_pass(K, S, same):
    """The shared-coefficient pass (operands of a domain held in registers over 16-row
    chunks; S = 150: ten chunks, the last partial) against the per-row pass over the
    same coefficient written out per domain: every output bit-identical, with the split
    term, the next layer's bias and the center sums all present."""
    dev = device()
    announce(f"shared-coefficient relax pass vs per-domain pass K={K} S={S} same={same}")
    g = torch.Generator().manual_seed(K * 7 + S)
    D = 5
    A_u = torch.randn(S, K, generator=g)
    A_l = A_u if same else torch.randn(S, K, generator=g)
    A_u[0, :3] = torch.tensor([0.0, -0.0, 1.0])
    l = torch.randn(D, K, generator=g)
    u = l + torch.rand(D, K, generator=g)
    alpha = torch.rand(D, K, generator=g)
    add = torch.randn(D, K, generator=g)
    kb = torch.randn(K, generator=g)
    cv = torch.randn(D, K, generator=g)
    bu, bl = torch.randn(D, S, generator=g), torch.randn(D, S, generator=g)
    d = {k: v.to(dev).contiguous() for k, v in dict(A_u=A_u, A_l=A_l, l=l, u=u, alpha=alpha, add=add, kb=kb, cv=cv,
                                                     bu=bu, bl=bl).items()}
    if same:
        d["A_l"] = d["A_u"]
    full_u = d["A_u"].expand(D, S, K).contiguous()
    full_l = full_u if same else d["A_l"].expand(D, S, K).contiguous()
    outs = []
    for Au, Al, stride in ((d["A_u"], d["A_l"], 0), (full_u, full_l, S * K)):
        o = [torch.empty(D * S, K, device=dev), torch.empty(D * S, K, device=dev)] + \
            [torch.empty(D * S, device=dev) for _ in range(4)]
        _lib.call("bf_crown_relu_relax_lu", _lib.ptr(Au), _lib.ptr(Al), stride, D, S, K, _lib.ptr(d["l"]),
                  _lib.ptr(d["u"]), _lib.ptr(d["alpha"]), K, _lib.ptr(d["add"]), K, _lib.ptr(d["kb"]),
                  _lib.ptr(d["cv"]), _lib.ptr(d["bu"]), _lib.ptr(d["bl"]), *[_lib.ptr(x) for x in o],
                  _lib.stream_handle())
        outs.append(o)
    torch.cuda.synchronize()
    for i, what in enumerate(("A_u'", "A_l'", "b_u", "b_l", "c_u", "c_l")):
        assert torch.equal(outs[0][i], outs[1][i]), what


@pytest.mark.parametrize("K,S,same", [(256, 9, False), (500, 9, True), (256, 20, False)])
def test_large_per_domain_pass_equals_per_row_pass(K, S, same):
    """A per-domain coefficient of at least 8192 rows (the domain's operands held in
    registers over its rows; S = 9: one workgroup of unequal waves per domain, S = 20: two
    chunks, the last partial) against the same rows relaxed in calls of fewer rows (the
    per-row pass): every output bit-identical, with the split term, the next layer's bias
    and the center sums present."""
    dev = device()
    announce(f"large per-domain relax pass vs per-row pass K={K} S={S} same={same}")
    g = torch.Generator().manual_seed(K * 5 + S)
    D = -(-8192 // S) + 3
    A_u = torch.randn(D, S, K, generator=g)
    A_l = A_u if same else torch.randn(D, S, K, generator=g)
    A_u[0, 0, :3] = torch.tensor([0.0, -0.0, 1.0])
    l = torch.randn(D, K, generator=g)
    u = l + torch.rand(D, K, generator=g)
    d = {k: v.to(dev).contiguous() for k, v in dict(A_u=A_u, A_l=A_l, l=l, u=u, alpha=torch.rand(D, K, generator=g),
                                                     add=torch.randn(D, K, generator=g), kb=torch.randn(K, generator=g),
                                                     cv=torch.randn(D, K, generator=g),
                                                     bu=torch.randn(D, S, generator=g),
                                                     bl=torch.randn(D, S, generator=g)).items()}
    if same:
        d["A_l"] = d["A_u"]

    def run(d0, d1):
        n = d1 - d0
        o = [torch.empty(n * S, K, device=dev), torch.empty(n * S, K, device=dev)] + \
            [torch.empty(n * S, device=dev) for _ in range(4)]
        Al = d["A_u"][d0:d1] if same else d["A_l"][d0:d1]
        _lib.call("bf_crown_relu_relax_lu", _lib.ptr(d["A_u"][d0:d1]), _lib.ptr(Al), S * K, n, S, K,
                  _lib.ptr(d["l"][d0:d1]), _lib.ptr(d["u"][d0:d1]), _lib.ptr(d["alpha"][d0:d1]), K,
                  _lib.ptr(d["add"][d0:d1]), K, _lib.ptr(d["kb"]), _lib.ptr(d["cv"][d0:d1]),
                  _lib.ptr(d["bu"][d0:d1]), _lib.ptr(d["bl"][d0:d1]), *[_lib.ptr(x) for x in o], _lib.stream_handle())
        return o

    whole = run(0, D)
    step = 8192 // S // 2
    parts = [run(a, min(a + step, D)) for a in range(0, D, step)]
    torch.cuda.synchronize()
    for i, what in enumerate(("A_u'", "A_l'", "b_u", "b_l", "c_u", "c_l")):
        assert torch.equal(whole[i], torch.cat([p[i] for p in parts])), what


# K = 133: scalar kernel (K % 4 != 0); 132, 256, 500: float4 kernel, a wave per row (500:
# two quad steps, the second partial); 2048, 4100: float4, a workgroup per row (4100: a
# partial last step); S = 19, 9, 3 vary the rows per domain
@pytest.mark.parametrize("K,S", [(133, 7), (132, 7), (2048, 7), (500, 19), (256, 9), (4100, 3)])
def test_relax_pass_and_dense_concretize_match_oracle(K, S):
    dev = device()
    announce(f"standalone relax pass + dense concretize K={K} S={S}")
    g = torch.Generator().manual_seed(11)
    D = 5
    A_u = torch.randn(D, S, K, generator=g)
    A_l = torch.randn(D, S, K, generator=g)
    A_u[0, 0, :4] = torch.tensor([0.0, -0.0, 1.0, -1.0])
    l = torch.randn(D, K, generator=g)
    u = l + torch.rand(D, K, generator=g)
    l[0, :3] = torch.tensor([0.0, -1.0, 0.0])
    u[0, :3] = torch.tensor([0.0, 0.0, 1.0])
    alpha = torch.rand(D, K, generator=g) * 1.4 - 0.2
    add = torch.randn(D, K, generator=g)
    bu, bl = torch.randn(D, S, generator=g), torch.randn(D, S, generator=g)
    pre = cr.IntervalState(l, u)
    ref = cr.relu_backward_dense(A_u, A_l, bu, bl, pre=pre, name="h", relu_alpha={"h": alpha},
                                 add_l={"h": add})
    d = [x.to(dev).contiguous() for x in (A_u, A_l, l, u, alpha, add, bu, bl)]
    out = [torch.empty(D * S, K, device=dev), torch.empty(D * S, K, device=dev), torch.empty(D * S, device=dev),
           torch.empty(D * S, device=dev)]
    table = torch.empty(D, K, 4, device=dev)
    _lib.call("bf_relu_relax_table", _lib.ptr(d[2]), _lib.ptr(d[3]), _lib.ptr(d[4]), K, D, K, _lib.ptr(table),
              _lib.stream_handle())
    _lib.call("bf_crown_relu_relax", _lib.ptr(d[0]), _lib.ptr(d[1]), S * K, D, S, K, _lib.ptr(table), _lib.ptr(d[5]), K,
              None, None, _lib.ptr(d[6]), _lib.ptr(d[7]), _lib.ptr(out[0]), _lib.ptr(out[1]), _lib.ptr(out[2]),
              _lib.ptr(out[3]), None, None, _lib.stream_handle())
    torch.cuda.synchronize()
    assert torch.equal(out[0].cpu().reshape(D, S, K), ref[0])
    assert torch.equal(out[1].cpu().reshape(D, S, K), ref[1])
    assert_bounds_close(out[2].reshape(D, S), ref[2], "relax b_u")
    assert_bounds_close(out[3].reshape(D, S), ref[3], "relax b_l")
    # dense Linf concretize of A_l
    x0 = torch.rand(D, K, generator=g)
    spec = cr.InputSpec.linf(value_name="input", center=x0, eps=0.05)
    lb_ref, ub_ref = cr.concretize_affine(spec, x0, cr.DenseOp(ref[1], (K,)), ref[3])
    lb = torch.empty(D * S, device=dev)
    xd = x0.to(dev).contiguous()
    Al = ref[1].to(dev).contiguous()
    bld = ref[3].to(dev).contiguous()
    _lib.call("bf_concretize_dense", _lib.ptr(Al), D, S, K, _lib.ptr(xd), None, 0.05, 0, _lib.ptr(bld), 1,
              _lib.ptr(lb), _lib.stream_handle())
    torch.cuda.synchronize()
    # fp32 cancellation in center - eps * norm + b: judged against the fp64 oracle where the fp32 one differs
    f = lambda x: x.double()
    spec64 = cr.InputSpec.linf(value_name="input", center=f(x0), eps=0.05)
    lb64, _ub64 = cr.concretize_affine(spec64, f(x0), cr.DenseOp(f(ref[1]), (K,)), f(ref[3]))
    assert_parity(lb.reshape(D, S), lb_ref, lb64, "concretize lb")


# (K, S, shared coefficient, alpha): float4 / scalar kernels, a wave or a workgroup per row,
# per-domain / shared / no lower-slope override, and no ReLU at all (identity)
@pytest.mark.parametrize("K,S,stride0,alpha_mode", [(132, 7, False, "domain"), (133, 7, False, "shared"),
                                                    (500, 19, True, "domain"), (2048, 3, False, "none"),
                                                    (256, 9, False, "identity")])
def test_relax_pass_from_box_equals_table_pass(K, S, stride0, alpha_mode):
    """bf_crown_relu_relax_lu computes the slopes from the pre-activation box with the
    arithmetic of bf_relu_relax_table: every output is bit-identical to the table pass."""
    dev = device()
    announce(f"relax pass from the box K={K} S={S} stride0={stride0} alpha={alpha_mode}")
    g = torch.Generator().manual_seed(K + S)
    D = 6
    A_u = torch.randn(S if stride0 else D * S, K, generator=g)
    A_l = A_u if stride0 else torch.randn(D * S, K, generator=g)
    l = torch.randn(D, K, generator=g)
    u = l + torch.rand(D, K, generator=g)
    l[0, :3] = torch.tensor([0.0, -1.0, 0.0])
    u[0, :3] = torch.tensor([0.0, 0.0, 1.0])
    alpha = {"domain": torch.rand(D, K, generator=g) * 1.4 - 0.2, "shared": torch.rand(K, generator=g)}.get(alpha_mode)
    alpha_ld = K if alpha_mode == "domain" else 0
    add = torch.randn(D, K, generator=g)
    kb = torch.randn(K, generator=g)
    cv = torch.randn(D, K, generator=g)
    b_in = torch.randn(D * S, generator=g)
    dd = lambda x: None if x is None else x.to(dev).contiguous()
    Au, Al, ld, ud, ad, addd, kbd, cvd, bd = (dd(x) for x in (A_u, A_l, l, u, alpha, add, kb, cv, b_in))
    if alpha_mode == "identity":
        ld = ud = ad = None
    stride = 0 if stride0 else S * K
    st = _lib.stream_handle()
    table = None
    if ld is not None:
        table = torch.empty(D, K, 4, device=dev)
        _lib.call("bf_relu_relax_table", _lib.ptr(ld), _lib.ptr(ud), _lib.ptr(ad), alpha_ld, D, K, _lib.ptr(table), st)
    outs = []
    for use_box in (False, True):
        o = [torch.empty(D * S, K, device=dev), torch.empty(D * S, K, device=dev)] + \
            [torch.empty(D * S, device=dev) for _ in range(4)]
        src = (_lib.ptr(ld), _lib.ptr(ud), _lib.ptr(ad), alpha_ld) if use_box else (_lib.ptr(table),)
        _lib.call("bf_crown_relu_relax_lu" if use_box else "bf_crown_relu_relax", _lib.ptr(Au), _lib.ptr(Al), stride,
                  D, S, K, *src, _lib.ptr(addd), K, _lib.ptr(kbd), _lib.ptr(cvd), _lib.ptr(bd), _lib.ptr(bd),
                  *(_lib.ptr(x) for x in o), st)
        outs.append(o)
    torch.cuda.synchronize()
    for i, (x, y) in enumerate(zip(*outs)):
        assert torch.equal(x.cpu(), y.cpu()), f"output {i} differs between the box and the table source"


def test_branch_update_matches_oracle():
    dev = device()
    announce("branch argmax update")
    g = torch.Generator().manual_seed(4)
    pre = {}
    for name, n in (("a", 70), ("b", 130)):
        l = torch.randn(33, n, generator=g)
        u = l + torch.rand(33, n, generator=g) * 2
        pre[name] = cr.IntervalState(l, u)
    # exact ties: row 0 -> two equal gaps inside "a", row 1 -> equal best gap in "a" and "b"
    pre["a"].lower[0, 5], pre["a"].upper[0, 5] = -3.0, 3.0
    pre["a"].lower[0, 9], pre["a"].upper[0, 9] = -2.0, 4.0
    pre["a"].lower[1, 2], pre["a"].upper[1, 2] = -4.0, 4.0
    pre["b"].lower[1, 1], pre["b"].upper[1, 1] = -5.0, 3.0
    pre["b"].lower[2] = 1.0  # no ambiguous neuron in layer b for row 2
    ref = ab.branch_choices(pre)
    gap = torch.full((33,), float("-inf"), device=dev)
    lay = torch.full((33,), -1, dtype=torch.int32, device=dev)
    idx = torch.zeros(33, dtype=torch.int32, device=dev)
    for li, (name, st) in enumerate(pre.items()):
        lo, hi = st.lower.to(dev).contiguous(), st.upper.to(dev).contiguous()
        _lib.call("bf_branch_update", _lib.ptr(lo), _lib.ptr(hi), 33, int(lo.shape[1]), li, _lib.ptr(gap),
                  _lib.ptr(lay), _lib.ptr(idx), _lib.stream_handle())
    names = list(pre.keys())
    got = [None if int(a) < 0 else (names[int(a)], int(b)) for a, b in zip(lay.cpu(), idx.cpu())]
    assert got == ref


def test_adam_clamp_matches_torch():
    dev = device()
    announce("adam + clamp step")
    g = torch.Generator().manual_seed(9)
    p0 = torch.rand(1000, generator=g)
    p = p0.clone().requires_grad_(True)
    opt = torch.optim.Adam([p], lr=0.2)
    pd = p0.to(dev).contiguous()
    m = torch.zeros_like(pd)
    v = torch.zeros_like(pd)
    for step in range(1, 6):
        grad = torch.randn(1000, generator=g) * (10.0 ** (step - 3))
        grad[:5] = 0.0
        opt.zero_grad()
        p.grad = grad.clone()
        opt.step()
        with torch.no_grad():
            p.clamp_(0.0, 1.0)
        gd = grad.to(dev).contiguous()
        _lib.call("bf_adam_clamp_step", _lib.ptr(pd), _lib.ptr(m), _lib.ptr(v), _lib.ptr(gd), 1000, 0.2, 0.9, 0.999,
                  1e-8, step, 0.0, 1.0, 1, _lib.stream_handle())
        torch.cuda.synchronize()
        # torch's CPU kernels mix fused and unfused multiply-adds; agree to a few ulps
        assert torch.allclose(pd.cpu(), p.detach(), rtol=1e-6, atol=1e-7), float((pd.cpu() - p.detach()).abs().max())


def _placed(t: torch.Tensor, offset: int) -> torch.Tensor:
    """A contiguous copy of ``t`` whose storage starts ``offset`` floats into a fresh buffer."""
    buf = torch.empty(t.numel() + offset, device=t.device, dtype=t.dtype)
    out = buf[offset:].view(t.shape)
    out.copy_(t)
    return out


@pytest.mark.parametrize("layout", ["ragged", "quad", "quad_misaligned"])
def test_multi_tensor_steps_equal_single_tensor_steps(layout):
    """bf_adam_clamp_multi (also with its fused best-of copy), bf_masked_copy_rows_multi and
    bf_beta_coeff_multi give, tensor by tensor, bit for bit what the single-tensor entry
    points give (18 tensors: two
    launches of the multi kernels; sizes not multiples of the workgroup).  "ragged":
    widths 3 + 41 i (the scalar path); "quad": widths that are multiples of 4 on
    16-byte-aligned storage (the float4 path of the best-of copy and the split term);
    "quad_misaligned": the same widths on storage one float off alignment (the scalar
    fallback)."""
    dev = device()
    announce(f"multi-tensor Adam / best-of copy / split term ({layout})")
    g = torch.Generator().manual_seed(21)
    st = _lib.stream_handle()
    D = 37
    cols = [3 + 41 * i for i in range(18)] if layout == "ragged" else [4 * (1 + 13 * i) for i in range(18)]
    off = 1 if layout == "quad_misaligned" else 0
    P = [_placed(torch.rand(D, c, generator=g).to(dev), off) for c in cols]
    G = [_placed(torch.randn(D, c, generator=g).to(dev), off) for c in cols]
    if layout == "quad":
        assert all(t.data_ptr() % 16 == 0 for t in P + G)
    if layout == "quad_misaligned":
        assert all(t.data_ptr() % 16 != 0 for t in P + G)
    clamps = [(0.0, 1.0) if i % 2 == 0 else (0.0, None) for i in range(len(cols))]
    P1 = [_placed(t, off) for t in P]
    M0 = [_placed(torch.zeros_like(t), off) for t in P]
    V0 = [_placed(torch.zeros_like(t), off) for t in P]
    M1 = [_placed(torch.zeros_like(t), off) for t in P]
    V1 = [_placed(torch.zeros_like(t), off) for t in P]
    for step in (1, 2, 3):
        for i, t in enumerate(P):
            lo, hi = clamps[i]
            _lib.call("bf_adam_clamp_step", _lib.ptr(t), _lib.ptr(M0[i]), _lib.ptr(V0[i]), _lib.ptr(G[i]), t.numel(),
                      0.2, 0.9, 0.999, 1e-8, step, lo, hi or 0.0, 0 if hi is None else 1, st)
        _lib.call("bf_adam_clamp_multi", len(P1), _lib.ptr_array(P1), _lib.ptr_array(M1), _lib.ptr_array(V1),
                  _lib.ptr_array(G), _lib.i64_array([t.numel() for t in P1]), _lib.f32_array([c[0] for c in clamps]),
                  _lib.f32_array([c[1] or 0.0 for c in clamps]), _lib.i32_array([0 if c[1] is None else 1 for c in clamps]),
                  0.2, 0.9, 0.999, 1e-8, step, None, None, 0, st)
    torch.cuda.synchronize()
    for i in range(len(P)):
        assert torch.equal(P[i], P1[i]) and torch.equal(M0[i], M1[i]) and torch.equal(V0[i], V1[i]), f"adam tensor {i}"
    mask = (torch.rand(D, generator=g) > 0.5).to(torch.int32).to(dev)
    dst0 = [_placed(torch.zeros_like(t), off) for t in P]
    dst1 = [_placed(torch.zeros_like(t), off) for t in P]
    for i, t in enumerate(P):
        _lib.call("bf_masked_copy_rows", _lib.ptr(dst0[i]), _lib.ptr(t), D, cols[i], _lib.ptr(mask), st)
    _lib.call("bf_masked_copy_rows_multi", len(P), _lib.ptr_array(dst1), _lib.ptr_array(P), _lib.i64_array(cols), D,
              _lib.ptr(mask), st)
    splits = [_placed(torch.randint(-1, 2, (D, c), generator=g, dtype=torch.int8).to(dev), 4 * off) for c in cols]
    out0 = [_placed(torch.empty_like(t), off) for t in P]
    out1 = [_placed(torch.empty_like(t), off) for t in P]
    for i, t in enumerate(P):
        _lib.call("bf_beta_coeff", _lib.ptr(t), cols[i], _lib.ptr(splits[i]), cols[i], D, cols[i], _lib.ptr(out0[i]), st)
    _lib.call("bf_beta_coeff_multi", len(P), _lib.ptr_array(P), _lib.i64_array(cols), _lib.ptr_array(splits),
              _lib.i64_array(cols), _lib.i64_array(cols), D, _lib.ptr_array(out1), st)
    torch.cuda.synchronize()
    for i in range(len(P)):
        assert torch.equal(dst0[i], dst1[i]), f"masked copy tensor {i}"
        assert torch.equal(out0[i], out1[i]), f"split term tensor {i}"
    # the best-of copy fused into the multi-tensor step: the masked rows get the values before the
    # step, and the step itself is the single-tensor one
    before = [t.clone() for t in P1]
    best = [_placed(torch.zeros_like(t), off) for t in P]
    for i, t in enumerate(P):
        lo, hi = clamps[i]
        _lib.call("bf_adam_clamp_step", _lib.ptr(t), _lib.ptr(M0[i]), _lib.ptr(V0[i]), _lib.ptr(G[i]), t.numel(),
                  0.2, 0.9, 0.999, 1e-8, 4, lo, hi or 0.0, 0 if hi is None else 1, st)
    _lib.call("bf_adam_clamp_multi", len(P1), _lib.ptr_array(P1), _lib.ptr_array(M1), _lib.ptr_array(V1),
              _lib.ptr_array(G), _lib.i64_array([t.numel() for t in P1]), _lib.f32_array([c[0] for c in clamps]),
              _lib.f32_array([c[1] or 0.0 for c in clamps]), _lib.i32_array([0 if c[1] is None else 1 for c in clamps]),
              0.2, 0.9, 0.999, 1e-8, 4, _lib.ptr_array(best), _lib.ptr(mask), D, st)
    torch.cuda.synchronize()
    keep = mask.bool()[:, None]
    for i in range(len(P)):
        assert torch.equal(P[i], P1[i]) and torch.equal(M0[i], M1[i]) and torch.equal(V0[i], V1[i]), f"adam tensor {i}"
        assert torch.equal(best[i], torch.where(keep, before[i], torch.zeros_like(before[i]))), f"best-of tensor {i}"


@pytest.mark.parametrize("with_alpha", [True, False])
def test_relu_grad_matches_formula(with_alpha):
    """bf_relu_grad (the reverse pass through one ReLU relaxation), on aligned storage and on
    storage one float off alignment (the same bits), against the gradient of the relaxed
    coefficient in float64: g_in = g * slope_sel + G * bias_sel, dL/dalpha = sum_s g * A over
    A >= 0 on passed ambiguous neurons, dL/dbeta = -split * sum_s g."""
    dev = device()
    announce(f"bf_relu_grad against its formula (alpha={with_alpha})")
    g = torch.Generator().manual_seed(33)
    D, S, N = 37, 9, 132
    c = torch.randn(D, N, generator=g)
    w = torch.rand(D, N, generator=g)
    lo, hi = c - w, c + 0.5 * w
    A = torch.randn(D * S, N, generator=g)
    go = torch.randn(D * S, N, generator=g)
    Gr = torch.randn(D * S, generator=g)
    alpha = (torch.rand(D, N, generator=g) * 1.2 - 0.1) if with_alpha else None
    split = torch.randint(-1, 2, (D, N), generator=g, dtype=torch.int8)
    st = _lib.stream_handle()
    outs = []
    for off in (0, 1):
        P = lambda x: None if x is None else _placed(x.to(dev), off if x.dtype != torch.int8 else 4 * off)  # noqa: E731
        t = {k: P(v) for k, v in dict(lo=lo, hi=hi, A=A, go=go, alpha=alpha, split=split).items()}
        Gd = Gr.to(dev)
        gin = _placed(torch.empty(D * S, N, device=dev), off)
        ga = _placed(torch.empty(D, N, device=dev), off)
        gb = _placed(torch.empty(D, N, device=dev), off)
        _lib.call("bf_relu_grad", _lib.ptr(t["go"]), _lib.ptr(t["A"]), S * N, D, S, N, _lib.ptr(t["lo"]),
                  _lib.ptr(t["hi"]), _lib.ptr(t["alpha"]), N if with_alpha else 0, _lib.ptr(Gd), _lib.ptr(t["split"]),
                  N, _lib.ptr(gin), _lib.ptr(ga), _lib.ptr(gb), st)
        outs.append((gin.cpu(), ga.cpu(), gb.cpu()))
    torch.cuda.synchronize()
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
    gin, ga, gb = outs[0]
    # the formulas in float64
    l64, u64 = lo.double(), hi.double()
    amb = (l64 < 0) & (u64 > 0)
    au = torch.where(u64 <= 0, 0.0, torch.where(l64 >= 0, 1.0, u64 / (u64 - l64).clamp_min(1.1920928955078125e-07)))
    bu = torch.where(amb, -l64 * au, 0.0)
    al = torch.where(u64 <= 0, 0.0, torch.where(l64 >= 0, 1.0, alpha.double().clamp(0, 1) if with_alpha else 0.0))
    A3, g3 = A.double().view(D, S, N), go.double().view(D, S, N)
    nn = A3 >= 0
    ref_in = torch.where(nn, g3 * al[:, None], g3 * au[:, None]) + Gr.double().view(D, S, 1) * torch.where(
        nn, 0.0, bu[:, None])
    assert torch.allclose(gin.double().view(D, S, N), ref_in, rtol=1e-5, atol=1e-6)
    passed = amb & ((alpha >= 0) & (alpha <= 1) if with_alpha else torch.zeros_like(amb))
    ref_ga = torch.where(passed, (torch.where(nn, g3 * A3, 0.0)).sum(1), 0.0)
    ref_gb = -split.double() * g3.sum(1)
    assert torch.allclose(ga.double(), ref_ga, rtol=1e-5, atol=1e-5)
    assert torch.allclose(gb.double(), ref_gb, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("relu", [0, 1])
def test_interval_center_radius_matches_torch(relu):
    """bf_interval_center_radius: (l + u) / 2 and (u - l) / 2 of the interval (of its ReLU
    when asked), bit for bit torch's fp32 arithmetic, either output alone when the other is
    NULL (the input concretization's box radius asks for the radius only)."""
    dev = device()
    announce(f"interval center/radius relu={relu}")
    g = torch.Generator().manual_seed(7 + relu)
    n = 100003
    lo = torch.randn(n, generator=g)
    hi = lo + torch.rand(n, generator=g)
    lo[:4] = torch.tensor([0.0, -0.0, -1.0, 2.0])
    hi[:4] = torch.tensor([0.0, 0.0, -0.5, 3.0])
    l, u = (lo.clamp_min(0), hi.clamp_min(0)) if relu else (lo, hi)
    d = [x.to(dev) for x in (lo, hi)]
    mid = torch.empty(n, device=dev)
    rad = torch.empty(n, device=dev)
    _lib.call("bf_interval_center_radius", _lib.ptr(d[0]), _lib.ptr(d[1]), n, relu, _lib.ptr(mid), _lib.ptr(rad),
              _lib.stream_handle())
    rad_only = torch.full((n,), 7.0, device=dev)
    _lib.call("bf_interval_center_radius", _lib.ptr(d[0]), _lib.ptr(d[1]), n, relu, None, _lib.ptr(rad_only),
              _lib.stream_handle())
    torch.cuda.synchronize()
    assert torch.equal(mid.cpu(), (l + u) / 2.0)
    assert torch.equal(rad.cpu(), (u - l) / 2.0)
    assert torch.equal(rad_only.cpu(), (u - l) / 2.0)


def test_flags_without_splits_are_zeros_made_on_read():
    """A forward trace with no split or constraint launches no flag fill (no box can be
    emptied); its ``infeasible`` reads as int32 zeros on the device, as the flags of a trace
    whose splits empty nothing."""
    dev = device()
    announce("forward trace flags without splits")
    w = wl.make_c1()
    wd = wl.to_device(w, dev)
    trace = hc.forward_ibp_trace(wd.module, wd.spec)
    assert trace.infeasible_flags is None
    flags = trace.infeasible
    assert flags.dtype == torch.int32 and flags.device.type == dev.type and tuple(flags.shape) == (w.batch,)
    assert int(flags.abs().sum()) == 0
    assert trace.infeasible is flags


def test_adam_first_step_does_not_read_the_moments():
    """At step 1 bf_adam_clamp_step and bf_adam_clamp_multi start the moments at zero
    (torch.optim.Adam's fresh state): NaN-filled m and v give the bits of zero-filled ones,
    and step 2 then reads the moments step 1 wrote."""
    dev = device()
    announce("Adam first step with unread moments")
    g = torch.Generator().manual_seed(3)
    p0 = torch.rand(3, 700, generator=g).to(dev)
    gr = [torch.randn(3, 700, generator=g).to(dev) for _ in range(2)]
    out = []
    for fill in (0.0, float("nan")):
        p, m, v = p0.clone(), torch.full_like(p0, fill), torch.full_like(p0, fill)
        q, mq, vq = p0.clone(), torch.full_like(p0, fill), torch.full_like(p0, fill)
        for step in (1, 2):
            _lib.call("bf_adam_clamp_step", _lib.ptr(p), _lib.ptr(m), _lib.ptr(v), _lib.ptr(gr[step - 1]), p.numel(),
                      0.1, 0.9, 0.999, 1e-8, step, 0.0, 1.0, 1, _lib.stream_handle())
            _lib.call("bf_adam_clamp_multi", 1, _lib.ptr_array([q]), _lib.ptr_array([mq]), _lib.ptr_array([vq]),
                      _lib.ptr_array([gr[step - 1]]), _lib.i64_array([q.numel()]), _lib.f32_array([0.0]),
                      _lib.f32_array([1.0]), _lib.i32_array([1]), 0.1, 0.9, 0.999, 1e-8, step, None, None, 0,
                      _lib.stream_handle())
        torch.cuda.synchronize()
        out.append((p, m, v, q, mq, vq))
    for a, b in zip(out[0], out[1]):
        assert torch.equal(a, b)
    assert torch.equal(out[0][0], out[0][3])
