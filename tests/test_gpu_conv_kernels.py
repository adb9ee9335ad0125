"""Direct parity of the conv kernels of the C ABI against float64 torch on the CPU.

bf_conv_transpose_rows replaces Conv2dLinearOperator.to_dense
(boundflow/runtime/linear_operator.py:1067-1092), i.e. conv_transpose2d of every
coefficient row, optionally fused with the concretization norm
sum |y| * w and the gradient seed h = h_scale * sign(y) * w.  Shapes with at
most 4 output channels and 16 taps run the tap-product MFMA kernel (in its register
form when the map has at most 16 channels and 256 pixels and each output pixel at
most 2 x 2 taps, else in its generic form), other
shapes with KH % sh == 0 and KW % sw == 0 the parity-class MFMA kernel, the
rest the row kernel; all three are covered, the parity-class kernel in both of its
map layouts (channel-last when Co is a multiple of 16).  bf_crown_relu_conv_transpose
(the ReLU relaxation applied while that kernel stages each row) is checked against
the relaxation pass followed by the transposed convolution.  bf_conv2d_rows (conv2d of rows with W or |W| and
a rank-1 term: the IBP conv step, the input-center projection and the gradient
of a transposed convolution) runs the same gather-GEMM kernel in its forward
mode.  Tolerance: the fp32 accumulation bound K * 2^-23 * sum |terms| of each
output (K = contributing taps).
"""

import pytest
import torch
import torch.nn.functional as F

from boundflow_amd import _lib
from tests.gpu_util import announce, device

pytestmark = pytest.mark.gpu

# (R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, S)
SHAPES = [
    (37, 32, 8, 8, 16, 4, 4, 2, 2, 1, 1, 9),     # C3 conv1 backward (channel-last parity-class MFMA kernel)
    (13, 16, 6, 6, 24, 2, 2, 2, 2, 0, 0, 3),     # one tap per class, 24 channels in two blocks (channel-last)
    (8, 48, 4, 4, 8, 3, 3, 1, 1, 1, 1, 4),       # stride 1, 9 taps, three 16-channel halves (channel-last)
    (20, 16, 16, 16, 3, 4, 4, 2, 2, 1, 1, 4),    # C3 conv0 backward (tap-product kernel, float4 map copy)
    (9, 8, 7, 5, 20, 3, 3, 1, 1, 1, 1, 3),       # stride 1, 3x3, Ci > 16 (parity-class kernel, 9 taps)
    (6, 5, 6, 6, 4, 2, 2, 2, 2, 0, 0, 2),        # 2x2 stride 2, no padding, 36 pixels (tap-product kernel)
    (7, 6, 5, 5, 3, 3, 3, 2, 2, 1, 1, 7),        # KH % sh != 0, 3 channels (tap-product kernel)
    (11, 7, 9, 9, 1, 3, 3, 1, 1, 0, 0, 4),       # one channel, stride 1, no padding (tap-product kernel, generic form)
    (600, 16, 16, 16, 3, 4, 4, 2, 2, 1, 1, 7),   # several rows per workgroup (tap-product kernel, register form)
    (5, 6, 5, 5, 8, 3, 3, 2, 2, 1, 1, 5),        # KH % sh != 0, 8 channels (row kernel)
]


def _out_hw(Ho, Wo, KH, KW, sh, sw, ph, pw):
    return (Ho - 1) * sh - 2 * ph + KH, (Wo - 1) * sw - 2 * pw + KW


@pytest.mark.parametrize("shape", SHAPES, ids=[f"R{s[0]}_Co{s[1]}_{s[2]}x{s[3]}_Ci{s[4]}_k{s[5]}s{s[7]}p{s[9]}"
                                                for s in SHAPES])
def test_conv_transpose_rows_matches_fp64(shape):
    dev = device()
    R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, S = shape
    Hi, Wi = _out_hw(Ho, Wo, KH, KW, sh, sw, ph, pw)
    announce(f"bf_conv_transpose_rows {shape} -> {Ci}x{Hi}x{Wi}")
    g = torch.Generator().manual_seed(R * 131 + Co)
    A_u = torch.randn(R, Co, Ho, Wo, generator=g)
    A_l = torch.randn(R, Co, Ho, Wo, generator=g)
    W = torch.randn(Co, Ci, KH, KW, generator=g)
    D = (R + S - 1) // S
    wv = torch.rand(D, Ci * Hi * Wi, generator=g)
    hsc = torch.randn(R, generator=g)
    ref = {k: F.conv_transpose2d(a.double(), W.double(), stride=(sh, sw), padding=(ph, pw))
           for k, a in (("u", A_u), ("l", A_l))}
    bound = {k: F.conv_transpose2d(a.double().abs(), W.double().abs(), stride=(sh, sw), padding=(ph, pw))
             for k, a in (("u", A_u), ("l", A_l))}
    taps = Co * ((KH + sh - 1) // sh) * ((KW + sw - 1) // sw)
    st = _lib.stream_handle()
    Ad = {k: v.to(dev) for k, v in (("u", A_u), ("l", A_l))}
    Wd, wvd, hsd = W.to(dev), wv.to(dev), hsc.to(dev)
    nout = Ci * Hi * Wi

    # store epilogue, both bounds
    y_u = torch.empty(R, Ci, Hi, Wi, device=dev)
    y_l = torch.empty(R, Ci, Hi, Wi, device=dev)
    _lib.call("bf_conv_transpose_rows", _lib.ptr(Ad["u"]), _lib.ptr(Ad["l"]), R, Co, Ho, Wo, _lib.ptr(Wd), Ci, KH,
              KW, sh, sw, ph, pw, Hi, Wi, _lib.ptr(y_u), _lib.ptr(y_l), S, None, 0, 0, None, None, None, None, st)
    # norm epilogue (Linf weights and box weights) with the gradient seed on the lower bound
    n_u = torch.empty(R, device=dev)
    n_l = torch.empty(R, device=dev)
    h = torch.empty(R, nout, device=dev)
    _lib.call("bf_conv_transpose_rows", _lib.ptr(Ad["u"]), _lib.ptr(Ad["l"]), R, Co, Ho, Wo, _lib.ptr(Wd), Ci, KH,
              KW, sh, sw, ph, pw, Hi, Wi, None, None, S, _lib.ptr(wvd), nout, 0, _lib.ptr(n_u), _lib.ptr(n_l),
              _lib.ptr(hsd), _lib.ptr(h), st)
    n1 = torch.empty(R, device=dev)
    _lib.call("bf_conv_transpose_rows", None, _lib.ptr(Ad["l"]), R, Co, Ho, Wo, _lib.ptr(Wd), Ci, KH, KW, sh, sw, ph,
              pw, Hi, Wi, None, None, S, None, 0, 0, None, _lib.ptr(n1), None, None, st)
    torch.cuda.synchronize()

    for k, y in (("u", y_u), ("l", y_l)):
        tol = taps * 2.0 ** -23 * bound[k] + 1e-30
        err = (y.cpu().double() - ref[k]).abs()
        assert bool((err <= tol).all()), f"y_{k}: {float((err / tol).max()):.3g} x tolerance"
    dom = torch.arange(R) // S
    wrow = wv.double()[dom].reshape(R, Ci, Hi, Wi)
    for k, n in (("u", n_u), ("l", n_l)):
        exact = (ref[k].abs() * wrow).flatten(1).sum(1)
        tol = (taps + nout) * 2.0 ** -23 * (bound[k] * wrow).flatten(1).sum(1)
        assert bool(((n.cpu().double() - exact).abs() <= tol).all()), f"norm_{k}"
    exact1 = ref["l"].abs().flatten(1).sum(1)
    tol1 = (taps + nout) * 2.0 ** -23 * bound["l"].flatten(1).sum(1)
    assert bool(((n1.cpu().double() - exact1).abs() <= tol1).all()), "Linf norm"
    # gradient seed: sign taken from the fp32 value; compare where |y| is above its rounding bound
    tol_l = (taps * 2.0 ** -23 * bound["l"]).flatten(1)
    sure = ref["l"].flatten(1).abs() > tol_l
    expect = hsc.double()[:, None] * torch.sign(ref["l"].flatten(1)) * wrow.flatten(1)
    got = h.cpu().double()
    assert torch.allclose(got[sure], expect[sure], rtol=1e-6, atol=0), "gradient seed"



@pytest.mark.parametrize("norm_p", [2, 1])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"R{s[0]}_Co{s[1]}_{s[2]}x{s[3]}_Ci{s[4]}_k{s[5]}s{s[7]}p{s[9]}"
                                                for s in SHAPES])
def test_conv_transpose_rows_lp_norms(shape, norm_p):
    """The L2 / L1 ball norms of each transposed-conv row in every kernel's epilogue:
    norm_p 2 gives sum y^2 (the root is the finalize's), norm_p 1 max |y|, for both
    bounds.  Tolerance: each y carries at most taps * 2^-23 * (|A| conv |W|); the sum
    of squares adds nout roundings, the max moves by at most the largest y error."""
    dev = device()
    R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, S = shape
    Hi, Wi = _out_hw(Ho, Wo, KH, KW, sh, sw, ph, pw)
    announce(f"bf_conv_transpose_rows Lp norm {norm_p} {shape}")
    g = torch.Generator().manual_seed(R * 17 + Co + norm_p)
    A = {k: torch.randn(R, Co, Ho, Wo, generator=g) for k in ("u", "l")}
    W = torch.randn(Co, Ci, KH, KW, generator=g)
    taps = Co * ((KH + sh - 1) // sh) * ((KW + sw - 1) // sw)
    nout = Ci * Hi * Wi
    n = {k: torch.full((R,), float("nan"), device=dev) for k in ("u", "l")}
    Ad, Wd = {k: v.to(dev) for k, v in A.items()}, W.to(dev)
    _lib.call("bf_conv_transpose_rows", _lib.ptr(Ad["u"]), _lib.ptr(Ad["l"]), R, Co, Ho, Wo,
              _lib.ptr(Wd), Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, None, None, S, None, 0, norm_p,
              _lib.ptr(n["u"]), _lib.ptr(n["l"]), None, None, _lib.stream_handle())
    torch.cuda.synchronize()
    for k in ("u", "l"):
        y = F.conv_transpose2d(A[k].double(), W.double(), stride=(sh, sw), padding=(ph, pw)).flatten(1)
        yb = F.conv_transpose2d(A[k].double().abs(), W.double().abs(), stride=(sh, sw), padding=(ph, pw)).flatten(1)
        if norm_p == 2:
            exact = y.pow(2).sum(1)
            tol = (2 * taps + nout) * 2.0 ** -23 * yb.pow(2).sum(1)
        else:
            exact = y.abs().amax(1)
            tol = taps * 2.0 ** -23 * yb.amax(1)
        err = (n[k].cpu().double() - exact).abs()
        assert bool((err <= tol + 1e-30).all()), f"norm_{k}: {float((err / tol).max()):.3g} x tolerance"
    # weights and gradient seeds belong to sum |y| only
    rc = _lib.load().bf_conv_transpose_rows(_lib.ptr(Ad["u"]), None, R, Co, Ho, Wo, _lib.ptr(Wd), Ci, KH, KW, sh, sw,
                                            ph, pw, Hi, Wi, None, None, S, _lib.ptr(Wd), 1, norm_p, _lib.ptr(n["u"]),
                                            None, None, None, _lib.stream_handle())
    assert rc != 0 and b"norm_p" in _lib.load().bf_last_error()

# (R, in_div, Ci, Hi, Wi, Co, KH, KW, sh, sw, ph, pw, abs_w, rank1)
CONV_SHAPES = [
    (40, 1, 16, 16, 16, 32, 4, 4, 2, 2, 1, 1, 0, True),    # C3 conv1 (gradient conv with the rank-1 term)
    (24, 1, 3, 32, 32, 16, 4, 4, 2, 2, 1, 1, 1, False),    # C3 conv0 radius (|W|)
    (18, 9, 3, 32, 32, 16, 4, 4, 2, 2, 1, 1, 0, False),    # center projection shared by 9 rows
    (7, 1, 20, 9, 7, 18, 3, 3, 1, 1, 1, 1, 0, True),       # 3x3 stride 1, Co > 16
]


@pytest.mark.parametrize("shape", CONV_SHAPES, ids=[f"R{s[0]}_div{s[1]}_Ci{s[2]}_{s[3]}x{s[4]}_Co{s[5]}_k{s[6]}s{s[8]}"
                                                      f"_abs{s[12]}_r1{int(s[13])}" for s in CONV_SHAPES])
def test_conv2d_rows_matches_fp64(shape):
    dev = device()
    R, in_div, Ci, Hi, Wi, Co, KH, KW, sh, sw, ph, pw, abs_w, rank1 = shape
    Ho = (Hi + 2 * ph - KH) // sh + 1
    Wo = (Wi + 2 * pw - KW) // sw + 1
    announce(f"bf_conv2d_rows {shape} -> {Co}x{Ho}x{Wo}")
    g = torch.Generator().manual_seed(R * 7 + Ci)
    nrows_in = (R + in_div - 1) // in_div
    x = torch.randn(nrows_in, Ci, Hi, Wi, generator=g)
    W = torch.randn(Co, Ci, KH, KW, generator=g)
    Wm = W.abs() if abs_w else W
    nout = Co * Ho * Wo
    rs = torch.randn(R, generator=g) if rank1 else None
    vdiv = 3
    vec = torch.randn((R + vdiv - 1) // vdiv, nout, generator=g) if rank1 else None
    xin = x.double()[torch.arange(R) // in_div]
    ref = F.conv2d(xin, Wm.double(), stride=(sh, sw), padding=(ph, pw)).reshape(R, nout)
    bound = F.conv2d(xin.abs(), W.double().abs(), stride=(sh, sw), padding=(ph, pw)).reshape(R, nout)
    if rank1:
        extra = rs.double()[:, None] * vec.double()[torch.arange(R) // vdiv]
        ref = ref + extra
        bound = bound + extra.abs()
    y = torch.empty(R, nout, device=dev)
    # device copies held by name until the kernel has run
    xd, Wd = x.to(dev), W.to(dev)
    rsd = None if rs is None else rs.to(dev)
    vd = None if vec is None else vec.to(dev)
    _lib.call("bf_conv2d_rows", _lib.ptr(xd), in_div, R, Ci, Hi, Wi, _lib.ptr(Wd), abs_w, Co, KH, KW,
              sh, sw, ph, pw, Ho, Wo, _lib.ptr(y), _lib.ptr(rsd), _lib.ptr(vd), vdiv if rank1 else 1,
              nout if rank1 else 0, _lib.stream_handle())
    torch.cuda.synchronize()
    tol = (Ci * KH * KW + 2) * 2.0 ** -23 * bound + 1e-30
    err = (y.cpu().double() - ref).abs()
    assert bool((err <= tol).all()), f"{float((err / tol).max()):.3g} x tolerance"


FUSED_SHAPES = [
    (37, 32, 8, 8, 16, 4, 4, 2, 2, 1, 1, 9),     # C3 / C4 conv1 region
    (8, 48, 4, 4, 8, 3, 3, 1, 1, 1, 1, 4),
]


@pytest.mark.parametrize("shape", FUSED_SHAPES, ids=[f"R{s[0]}_Co{s[1]}_Ci{s[4]}" for s in FUSED_SHAPES])
@pytest.mark.parametrize("variant", ["crown", "alpha_split"])
def test_relu_conv_transpose_matches_pass_then_conv(shape, variant):
    """bf_crown_relu_conv_transpose against bf_crown_relu_relax_lu + a float64 conv_transpose2d:
    the relaxed rows it writes are bit-identical to the pass's, the bias rows agree to the
    fp32 bound of their two summation orders, and y to the accumulation bound of the
    transposed convolution of those rows."""
    dev = device()
    R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, S = shape
    Hi, Wi = _out_hw(Ho, Wo, KH, KW, sh, sw, ph, pw)
    announce(f"bf_crown_relu_conv_transpose {shape} {variant}")
    assert _lib.load().bf_conv_transpose_hwc_supported(Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi) == 1
    g = torch.Generator().manual_seed(R * 7 + Co)
    D = (R + S - 1) // S
    R = D * S
    nin = Co * Ho * Wo
    A_u = torch.randn(R, nin, generator=g)
    A_l = torch.randn(R, nin, generator=g)
    c = torch.randn(D, nin, generator=g)
    w = torch.rand(D, nin, generator=g)
    lo, hi = c - w, c + 0.5 * w          # mixes inactive, active and ambiguous neurons
    W = torch.randn(Co, Ci, KH, KW, generator=g)
    kb = torch.randn(nin, generator=g)
    b_in = torch.randn(2, R, generator=g)
    alpha = torch.rand(D, nin, generator=g) if variant == "alpha_split" else None
    add = torch.randn(D, nin, generator=g) if variant == "alpha_split" else None
    T = lambda x: None if x is None else x.to(dev).contiguous()   # noqa: E731
    st = _lib.stream_handle()
    args = dict(A_u=T(A_u), A_l=T(A_l), lo=T(lo), hi=T(hi), alpha=T(alpha), add=T(add), kb=T(kb), bu=T(b_in[0]),
                bl=T(b_in[1]), W=T(W))
    # the pass, then the transposed convolution of its output in float64
    rp_u = torch.empty(R, nin, device=dev)
    rp_l = torch.empty(R, nin, device=dev)
    bp_u = torch.empty(R, device=dev)
    bp_l = torch.empty(R, device=dev)
    _lib.call("bf_crown_relu_relax_lu", _lib.ptr(args["A_u"]), _lib.ptr(args["A_l"]), S * nin, D, S, nin,
              _lib.ptr(args["lo"]), _lib.ptr(args["hi"]), _lib.ptr(args["alpha"]), nin if alpha is not None else 0,
              _lib.ptr(args["add"]), nin, _lib.ptr(args["kb"]), None, _lib.ptr(args["bu"]), _lib.ptr(args["bl"]),
              _lib.ptr(rp_u), _lib.ptr(rp_l), _lib.ptr(bp_u), _lib.ptr(bp_l), None, None, st)
    # the fused pass
    geo = (Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi)
    packed = torch.empty(int(_lib.load().bf_conv_transpose_packed_floats(*geo)), device=dev)
    _lib.call("bf_conv_transpose_pack_weights", _lib.ptr(args["W"]), *geo, _lib.ptr(packed), st)
    outs = []
    for wp in (None, packed):   # weights gathered by each workgroup, then the packed copy
        y_u = torch.empty(R, Ci * Hi * Wi, device=dev)
        y_l = torch.empty(R, Ci * Hi * Wi, device=dev)
        b_u = torch.empty(R, device=dev)
        b_l = torch.empty(R, device=dev)
        rf_l = torch.empty(R, nin, device=dev)
        _lib.call("bf_crown_relu_conv_transpose", _lib.ptr(args["A_u"]), _lib.ptr(args["A_l"]), D, S, Co, Ho, Wo,
                  _lib.ptr(args["lo"]), _lib.ptr(args["hi"]), _lib.ptr(args["alpha"]), nin if alpha is not None else 0,
                  _lib.ptr(args["add"]), nin, _lib.ptr(args["kb"]), _lib.ptr(args["bu"]), _lib.ptr(args["bl"]),
                  _lib.ptr(args["W"]), _lib.ptr(wp), Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, _lib.ptr(y_u), _lib.ptr(y_l),
                  _lib.ptr(b_u), _lib.ptr(b_l), None, _lib.ptr(rf_l), st)
        outs.append((y_u, y_l, b_u, b_l, rf_l))
    torch.cuda.synchronize()
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b), "packed weights change the result"
    y_u, y_l, b_u, b_l, rf_l = outs[1]
    assert torch.equal(rf_l, rp_l), "relaxed rows differ from the relaxation pass"
    for k, rp, y, bf, bp, A in (("u", rp_u, y_u, b_u, bp_u, A_u), ("l", rp_l, y_l, b_l, bp_l, A_l)):
        ref = F.conv_transpose2d(rp.double().cpu().reshape(R, Co, Ho, Wo), W.double(), stride=(sh, sw),
                                 padding=(ph, pw)).reshape(R, -1)
        bound = F.conv_transpose2d(rp.double().cpu().abs().reshape(R, Co, Ho, Wo), W.double().abs(),
                                   stride=(sh, sw), padding=(ph, pw)).reshape(R, -1)
        taps = Co * ((KH + sh - 1) // sh) * ((KW + sw - 1) // sw)
        err = (y.double().cpu() - ref).abs()
        assert bool((err <= taps * 2.0 ** -23 * bound + 1e-30).all()), f"y_{k}: max err {float(err.max()):.3e}"
        # bias rows: the same terms summed in two orders; bound 2 * nin * u * sum |terms|
        beta_max = float(lo.abs().max())   # every intercept -l u / (u - l) of an ambiguous neuron is at most |l|
        terms = (A.abs().sum(1).double() * beta_max + rp.double().cpu().abs().mul(kb.double().abs()).sum(1)
                 + float(b_in.abs().max()))
        berr = (bf.double().cpu() - bp.double().cpu()).abs()
        assert bool((berr <= 2 * nin * 2.0 ** -24 * terms + 1e-30).all()), f"b_{k}: max err {float(berr.max()):.3e}"


INPUT_SHAPES = [
    (37, 16, 16, 16, 3, 4, 4, 2, 2, 1, 1, 9),    # C3 / C4 input region (3 channels, 4 x 4 taps, stride 2)
    (10, 8, 6, 6, 2, 3, 3, 1, 1, 1, 1, 5),       # npix % 16 != 0: the scalar staging path (generic form)
    (603, 16, 16, 16, 3, 4, 4, 2, 2, 1, 1, 7),   # several rows per workgroup, domains changing inside one
    (40, 8, 14, 14, 1, 4, 4, 2, 2, 1, 1, 5),     # one output channel of 28 x 28, 196 map pixels (partial blocks)
    (20, 12, 8, 8, 4, 3, 3, 2, 2, 1, 1, 4),      # four output channels, 3 x 3 taps at stride 2 (absent taps)
]


@pytest.mark.parametrize("shape", INPUT_SHAPES, ids=[f"R{s[0]}_Co{s[1]}_Ci{s[4]}" for s in INPUT_SHAPES])
@pytest.mark.parametrize("variant", ["linf", "box_alpha_split", "l2", "l1"])
def test_relu_conv_transpose_concretize_matches_pass_then_conv(shape, variant):
    """bf_crown_relu_conv_transpose_concretize (the input layer in one pass) against
    bf_crown_relu_relax_lu + bf_conv_transpose_rows with norm outputs: the relaxed rows
    bit-identical to the pass's, the bias and center sums within the fp32 bound of their
    two summation orders, the norms within the accumulation bound of the transposed
    convolution, and the gradient seed equal where the sign of y is certain.  l2 / l1:
    the norms of the L2 / L1 ball (sum y^2, max |y|), without the gradient seed."""
    dev = device()
    R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, S = shape
    Hi, Wi = _out_hw(Ho, Wo, KH, KW, sh, sw, ph, pw)
    announce(f"bf_crown_relu_conv_transpose_concretize {shape} {variant}")
    assert _lib.load().bf_conv_transpose_small_supported(Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi) == 1
    g = torch.Generator().manual_seed(R * 5 + Co)
    D = (R + S - 1) // S
    R = D * S
    nin, nout = Co * Ho * Wo, Ci * Hi * Wi
    A_u = torch.randn(R, nin, generator=g)
    A_l = torch.randn(R, nin, generator=g)
    c = torch.randn(D, nin, generator=g)
    w = torch.rand(D, nin, generator=g)
    lo, hi = c - w, c + 0.5 * w
    W = torch.randn(Co, Ci, KH, KW, generator=g)
    kb = torch.randn(nin, generator=g)
    cv = torch.randn(D, nin, generator=g)
    b_in = torch.randn(2, R, generator=g)
    box = variant.startswith("box")
    alpha = torch.rand(D, nin, generator=g) if box else None
    add = torch.randn(D, nin, generator=g) if box else None
    wv = torch.rand(D, nout, generator=g) if box else None
    norm_p = {"l2": 2, "l1": 1}.get(variant, 0)
    h_scale = torch.randn(R, generator=g) if norm_p == 0 else None
    T = lambda x: None if x is None else x.to(dev).contiguous()   # noqa: E731
    a = {k: T(v) for k, v in dict(A_u=A_u, A_l=A_l, lo=lo, hi=hi, alpha=alpha, add=add, kb=kb, cv=cv, bu=b_in[0],
                                  bl=b_in[1], W=W, wv=wv, hs=h_scale).items()}
    P = lambda k: _lib.ptr(a[k])   # noqa: E731
    st = _lib.stream_handle()
    ald = nin if alpha is not None else 0
    # the pass, then the transposed conv with norm outputs
    rp = [torch.empty(R, nin, device=dev) for _ in range(2)]
    bp = [torch.empty(R, device=dev) for _ in range(2)]
    cp = [torch.empty(R, device=dev) for _ in range(2)]
    _lib.call("bf_crown_relu_relax_lu", P("A_u"), P("A_l"), S * nin, D, S, nin, P("lo"), P("hi"), P("alpha"), ald,
              P("add"), nin, P("kb"), P("cv"), P("bu"), P("bl"), _lib.ptr(rp[0]), _lib.ptr(rp[1]), _lib.ptr(bp[0]),
              _lib.ptr(bp[1]), _lib.ptr(cp[0]), _lib.ptr(cp[1]), st)
    np_ = [torch.empty(R, device=dev) for _ in range(2)]
    hp = torch.empty(R, nout, device=dev) if norm_p == 0 else None
    _lib.call("bf_conv_transpose_rows", _lib.ptr(rp[0]), _lib.ptr(rp[1]), R, Co, Ho, Wo, P("W"), Ci, KH, KW, sh, sw,
              ph, pw, Hi, Wi, None, None, S, P("wv"), nout, norm_p, _lib.ptr(np_[0]), _lib.ptr(np_[1]), P("hs"),
              _lib.ptr(hp), st)
    # the fused kernel
    nf = [torch.empty(R, device=dev) for _ in range(2)]
    bf = [torch.empty(R, device=dev) for _ in range(2)]
    cf = [torch.empty(R, device=dev) for _ in range(2)]
    hf = torch.empty(R, nout, device=dev) if norm_p == 0 else None
    rf_l = torch.empty(R, nin, device=dev)
    eps = 1.0 if box else 0.7
    lbf, ubf = torch.empty(R, device=dev), torch.empty(R, device=dev)
    _lib.call("bf_crown_relu_conv_transpose_concretize", P("A_u"), P("A_l"), D, S, Co, Ho, Wo, P("lo"), P("hi"),
              P("alpha"), ald, P("add"), nin, P("kb"), P("cv"), P("bu"), P("bl"), P("W"), Ci, KH, KW, sh, sw, ph, pw,
              Hi, Wi, P("wv"), nout, norm_p, P("hs"), _lib.ptr(hf), _lib.ptr(nf[0]), _lib.ptr(nf[1]), _lib.ptr(bf[0]),
              _lib.ptr(bf[1]), _lib.ptr(cf[0]), _lib.ptr(cf[1]), None, _lib.ptr(rf_l), eps, _lib.ptr(lbf),
              _lib.ptr(ubf), st)
    # the bounds the launch wrote are the finalize's of its own norms, centers and biases, bit for bit
    lb_ref, ub_ref = torch.empty(R, device=dev), torch.empty(R, device=dev)
    _lib.call("bf_concretize_finalize", _lib.ptr(nf[0]), _lib.ptr(nf[1]), 1, R, _lib.ptr(cf[0]), _lib.ptr(cf[1]),
              _lib.ptr(bf[0]), _lib.ptr(bf[1]), eps, norm_p, _lib.ptr(lb_ref), _lib.ptr(ub_ref), st)
    torch.cuda.synchronize()
    assert torch.equal(lbf, lb_ref) and torch.equal(ubf, ub_ref), "bounds differ from the finalize of the norms"
    assert torch.equal(rf_l, rp[1]), "relaxed rows differ from the relaxation pass"
    beta_max = float(lo.abs().max())
    for z, A in ((0, A_u), (1, A_l)):
        rel = rp[z].double().cpu()
        y = F.conv_transpose2d(rel.reshape(R, Co, Ho, Wo), W.double(), stride=(sh, sw), padding=(ph, pw)).reshape(R, -1)
        ybound = F.conv_transpose2d(rel.abs().reshape(R, Co, Ho, Wo), W.double().abs(), stride=(sh, sw),
                                    padding=(ph, pw)).reshape(R, -1)
        taps = Co * ((KH + sh - 1) // sh) * ((KW + sw - 1) // sw)
        wgt = wv.double()[torch.arange(R) // S] if box else torch.ones(R, nout, dtype=torch.float64)
        ytol = taps * 2.0 ** -23 * ybound
        if norm_p == 2:
            nref = y.pow(2).sum(1)
            ntol = (2 * taps + nout) * 2.0 ** -23 * ybound.pow(2).sum(1) + 1e-30
        elif norm_p == 1:
            nref = y.abs().amax(1)
            ntol = ytol.amax(1) + 1e-30
        else:
            nref = (y.abs() * wgt).sum(1)
            ntol = (ytol * wgt).sum(1) + nout * 2.0 ** -23 * nref + 1e-30
        nerr = (nf[z].double().cpu() - nref).abs()
        assert bool((nerr <= ntol).all()), f"norm {z}: {float((nerr / ntol).max()):.3g} x tolerance"
        terms = (A.abs().sum(1).double() * beta_max + rel.abs().mul(kb.double().abs()).sum(1)
                 + float(b_in.abs().max()))
        berr = (bf[z].double().cpu() - bp[z].double().cpu()).abs()
        assert bool((berr <= 2 * nin * 2.0 ** -24 * terms + 1e-30).all()), f"b {z}: max err {float(berr.max()):.3e}"
        cterms = (rel.abs() * cv.double().abs()[torch.arange(R) // S]).sum(1)
        cerr = (cf[z].double().cpu() - cp[z].double().cpu()).abs()
        assert bool((cerr <= 2 * nin * 2.0 ** -24 * cterms + 1e-30).all()), f"c {z}: max err {float(cerr.max()):.3e}"
        if z == 1 and norm_p == 0:
            sure = y.abs() > ytol
            assert torch.equal(hf.cpu()[sure], hp.cpu()[sure]), "gradient seed differs where sign(y) is certain"
