"""The contraction's 64 x 128 tile configuration (TileQ, 6 workgroups per CU), taken
by plain-prologue contractions whose 128 x 128 tiles would load the 256 CUs
unevenly (C5's 36 864-row grids): the store, rank-1 store and |A W|
concretization epilogues against float64 on shapes that select it, with row,
column and K tails.  The relaxation epilogue on such a shape is covered by
test_gpu_epilogue_relax.test_two_region_step_matches_oracle (D = 2048).  The 64 x 64
TileS (plain-prologue store contractions on grids of fewer 128 x 128 tiles than
CUs): plain, two-sided, rank-1 and split-K forms against float64."""

import pytest
import torch

from boundflow_amd import _lib
from tests.gpu_util import announce, contraction_tol, device

pytestmark = pytest.mark.gpu


def tile(M, N, nz=1):
    return chr(_lib.load().bf_gemm_tile_config(M, N, nz, 1, 0, 1))


@pytest.mark.parametrize("M,N,K,abs_b", [(16512, 256, 256, 0), (16500, 250, 260, 1), (36864, 256, 256, 0)])
def test_store_on_tile_q_matches_fp64(M, N, K, abs_b):
    dev = device()
    announce(f"gemm on TileQ M={M} N={N} K={K} abs_b={abs_b}")
    assert tile(M, N) == "Q"
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(M, K, generator=g)
    B = torch.randn(N, K, generator=g)
    Bm = B.t().abs() if abs_b else B.t()
    ref = A.double() @ Bm.double()
    C = torch.empty(M, N, device=dev)
    Ad, Bd = A.to(dev), B.to(dev)
    _lib.call("bf_gemm", _lib.ptr(Ad), K, _lib.ptr(Bd), K, 1, abs_b, _lib.ptr(C), N, M, N, K, _lib.stream_handle())
    torch.cuda.synchronize()
    tol = contraction_tol(A, Bm, K) + 1e-30
    err = (C.cpu().double() - ref).abs()
    assert bool((err <= tol).all()), float((err / tol).max())


def test_rank1_store_on_tile_q_matches_fp64():
    """C5's gradient contraction shape: g . W^T + r_row x v_col[d] (9 rows per domain)."""
    dev = device()
    M, N, K, S = 36864, 256, 256, 9
    announce(f"gemm_rank1 on TileQ M={M} N={N} K={K} S={S}")
    assert tile(M, N) == "Q"
    g = torch.Generator().manual_seed(5)
    A = torch.randn(M, K, generator=g)
    W = torch.randn(N, K, generator=g)
    r = torch.randn(M, generator=g)
    v = torch.randn(M // S, N, generator=g)
    rv = r.double()[:, None] * v.double()[torch.arange(M) // S]
    ref = A.double() @ W.double().t() + rv
    tol = contraction_tol(A, W.t(), K) + rv.abs() * 2.0 ** -22
    C = torch.empty(M, N, device=dev)
    Ad, Wd, rd, vd = A.to(dev), W.to(dev), r.to(dev), v.to(dev)
    _lib.call("bf_gemm_rank1", _lib.ptr(Ad), K, _lib.ptr(Wd), K, 1, _lib.ptr(C), N, M, N, K, S, _lib.ptr(rd),
              _lib.ptr(vd), N, None, 0, _lib.stream_handle())
    torch.cuda.synchronize()
    err = (C.cpu().double() - ref).abs()
    assert bool((err <= tol).all()), float((err / tol).max())


@pytest.mark.parametrize("box", [False, True])
def test_concretize_on_tile_q_matches_fp64(box):
    """bf_crown_linear_concretize (|A W| row sums, weighted by the box radius for a
    box, and the gradient seed h = h_scale * sign(A W) (* radius)) for both bounds
    of 2048 domains x 9 rows."""
    dev = device()
    D, S, N, I = 2048, 9, 256, 252
    M = D * S
    announce(f"concretize on TileQ D={D} S={S} N={N} I={I} box={box}")
    assert tile(M, I, 2) == "Q"
    g = torch.Generator().manual_seed(11 + box)
    A_u = torch.randn(M, N, generator=g)
    A_l = torch.randn(M, N, generator=g)
    Wt = torch.randn(I, N, generator=g) * 0.1          # [I, N]: C = A @ Wt^T
    rad = torch.rand(D, I, generator=g) if box else None
    eps = 1.0 if box else 0.05
    cen_u, cen_l = torch.randn(M, generator=g), torch.randn(M, generator=g)
    b_u, b_l = torch.randn(M, generator=g), torch.randn(M, generator=g)
    h_scale = torch.randn(M, generator=g)
    w64 = rad.double()[torch.arange(M) // S] if box else torch.ones(M, I, dtype=torch.float64)
    refs = {}
    for side, A, cen, b in (("u", A_u, cen_u, b_u), ("l", A_l, cen_l, b_l)):
        C = A.double() @ Wt.double().t()
        nrm = (C.abs() * w64).sum(1)
        val = cen.double() + (eps * nrm if side == "u" else -eps * nrm) + b.double()
        tolC = contraction_tol(A, Wt.t(), N)
        tol = eps * ((tolC * w64).sum(1) + I * 2.0 ** -23 * nrm) + 2.0 ** -22 * (cen.double().abs() + b.double().abs()
                                                                                 + eps * nrm)
        refs[side] = (C, val, tol, tolC)
    d = lambda x: None if x is None else x.to(dev).contiguous()
    ws = torch.empty(int(_lib.load().bf_crown_linear_concretize_workspace(D, S, I)), device=dev)
    lb, ub = torch.empty(M, device=dev), torch.empty(M, device=dev)
    h_out = torch.empty(M, I, device=dev)
    A_ud, A_ld, Wtd, radd = d(A_u), d(A_l), d(Wt), d(rad)
    _lib.call("bf_crown_linear_concretize", _lib.ptr(A_ud), _lib.ptr(A_ld), S * N, D, S, N, _lib.ptr(Wtd), I,
              _lib.ptr(radd), eps, 0, _lib.ptr(d(cen_u)), _lib.ptr(d(cen_l)), _lib.ptr(d(b_u)), _lib.ptr(d(b_l)),
              _lib.ptr(d(h_scale)), _lib.ptr(h_out), _lib.ptr(ws), _lib.ptr(lb), _lib.ptr(ub), _lib.stream_handle())
    torch.cuda.synchronize()
    for side, got in (("u", ub), ("l", lb)):
        _C, val, tol, _t = refs[side]
        err = (got.cpu().double() - val).abs()
        announce(f"  {side}: max abs err {float(err.max()):.3e}")
        assert bool((err <= tol).all()), f"{side}: {float((err / tol).max()):.3f} x tolerance"
    # gradient seed of the lower bound: exact where the product's sign is certain
    C_l, _v, _t, tolC = refs["l"]
    sure = C_l.abs() > tolC
    h_ref = h_scale.double()[:, None] * torch.sign(C_l) * w64
    got = h_out.cpu().double()
    assert torch.equal(got[sure], h_ref[sure].float().double())


@pytest.mark.parametrize("M,N,K,trans_b", [(288, 2048, 100, 1), (300, 250, 77, 1), (130, 70, 33, 0)])
def test_store_on_tile_s_matches_fp64(M, N, K, trans_b):
    """Grids of fewer 128 x 128 tiles than CUs with the plain prologue (the CNN
    configurations' fully connected layers) run on the 64 x 64 TileS: row, column and
    K tails, either B layout."""
    dev = device()
    announce(f"gemm on TileS M={M} N={N} K={K} trans_b={trans_b}")
    assert tile(M, N, 1) == "S"
    g = torch.Generator().manual_seed(M * 7 + N + K)
    A = torch.randn(M, K, generator=g)
    B = torch.randn(N, K, generator=g) if trans_b else torch.randn(K, N, generator=g)
    Bm = B.t() if trans_b else B
    ref = A.double() @ Bm.double()
    C = torch.empty(M, N, device=dev)
    Ad, Bd = A.to(dev), B.contiguous().to(dev)
    ldb = K if trans_b else N
    _lib.call("bf_gemm", _lib.ptr(Ad), K, _lib.ptr(Bd), ldb, trans_b, 0, _lib.ptr(C), N, M, N, K, _lib.stream_handle())
    torch.cuda.synchronize()
    tol = contraction_tol(A, Bm, K) + 1e-30
    err = (C.cpu().double() - ref).abs()
    assert bool((err <= tol).all()), float((err / tol).max())


@pytest.mark.parametrize("form", ["nz2_store", "rank1_S9", "rank1_split_k", "rank1_small_out"])
def test_other_store_forms_on_tile_s_match_fp64(form):
    """The other plain-prologue store forms that take TileS on small grids: both
    coefficient sides in one launch (bf_crown_relu_linear_fwd with nothing to relax,
    nz = 2), the rank-1 epilogue with 9 rows per domain (bf_gemm_rank1, S = 9), the
    rank-1 epilogue with K split into chunks summed by splitk_reduce, and a small output
    whose split K takes the one-launch small-output kernel (rank-1 term in its epilogue)."""
    dev = device()
    g = torch.Generator().manual_seed({"nz2_store": 3, "rank1_S9": 4, "rank1_split_k": 5, "rank1_small_out": 6}[form])
    st = _lib.stream_handle()
    if form == "nz2_store":
        D, S, N, P = 32, 9, 256, 100
        M = D * S
        announce(f"crown_relu_linear_fwd (plain, nz=2) on TileS M={M} N={P} K={N}")
        assert tile(M, P, 2) == "S"
        A_u, A_l = torch.randn(M, N, generator=g), torch.randn(M, N, generator=g)
        W = torch.randn(P, N, generator=g)
        b_u, b_l = torch.randn(M, generator=g), torch.randn(M, generator=g)
        d = {k: v.to(dev) for k, v in dict(A_u=A_u, A_l=A_l, W=W, b_u=b_u, b_l=b_l).items()}
        out_u, out_l = torch.empty(M, P, device=dev), torch.empty(M, P, device=dev)
        bo_u, bo_l = torch.empty(M, device=dev), torch.empty(M, device=dev)
        _lib.call("bf_crown_relu_linear_fwd", _lib.ptr(d["A_u"]), _lib.ptr(d["A_l"]), S * N, D, S, N, None, None, 0,
                  _lib.ptr(d["W"]), P, 1, None, _lib.ptr(d["b_u"]), _lib.ptr(d["b_l"]), _lib.ptr(out_u),
                  _lib.ptr(out_l), _lib.ptr(bo_u), _lib.ptr(bo_l), st)
        torch.cuda.synchronize()
        for A, out, b_in, b_out in ((A_u, out_u, b_u, bo_u), (A_l, out_l, b_l, bo_l)):
            ref = A.double() @ W.double().t()
            tol = contraction_tol(A, W.t(), N) + 1e-30
            err = (out.cpu().double() - ref).abs()
            assert bool((err <= tol).all()), float((err / tol).max())
            assert torch.equal(b_out.cpu(), b_in), "b_out is b_in when nothing is relaxed"
        return
    # rank1_S9: an unsplit TileS contraction (K = 200 below the split threshold); rank1_split_k: an output of
    # more than 1024 tiles of 16 x 16 whose K is split over TileS chunks and reduced in chunk order;
    # rank1_small_out: a small output whose split K takes the one-launch small-output kernel instead
    M, N, K, S = {"rank1_S9": (288, 100, 200, 9), "rank1_split_k": (1152, 400, 1024, 9),
                  "rank1_small_out": (288, 100, 1024, 9)}[form]
    ws_floats = int(_lib.load().bf_gemm_rank1_workspace(M, N, K))
    if form in ("rank1_split_k", "rank1_small_out"):
        assert ws_floats > 0, "this shape splits K"
        assert (-(-M // 16) * -(-N // 16) > 1024) == (form == "rank1_split_k")
    else:
        # K below the split threshold: the contraction runs unsplit on TileS
        assert ws_floats == 0
        assert tile(M, N) == "S"
    announce(f"gemm_rank1 {form} M={M} N={N} K={K} S={S} workspace={ws_floats}")
    A = torch.randn(M, K, generator=g)
    W = torch.randn(N, K, generator=g)
    r = torch.randn(M, generator=g)
    v = torch.randn(M // S, N, generator=g)
    rv = r.double()[:, None] * v.double()[torch.arange(M) // S]
    ref = A.double() @ W.double().t() + rv
    tol = contraction_tol(A, W.t(), K) + rv.abs() * 2.0 ** -22 + 1e-30
    C = torch.empty(M, N, device=dev)
    ws = torch.empty(max(ws_floats, 1), device=dev)
    Ad, Wd, rd, vd = A.to(dev), W.to(dev), r.to(dev), v.to(dev)
    _lib.call("bf_gemm_rank1", _lib.ptr(Ad), K, _lib.ptr(Wd), K, 1, _lib.ptr(C), N, M, N, K, S, _lib.ptr(rd),
              _lib.ptr(vd), N, _lib.ptr(ws) if ws_floats else None, ws_floats, st)
    torch.cuda.synchronize()
    err = (C.cpu().double() - ref).abs()
    assert bool((err <= tol).all()), float((err / tol).max())
