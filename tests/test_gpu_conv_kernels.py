"""Direct parity of the conv kernels of the C ABI against float64 torch on the CPU.

bf_conv_transpose_rows replaces Conv2dLinearOperator.to_dense
(boundflow/runtime/linear_operator.py:1067-1092), i.e. conv_transpose2d of every
coefficient row, optionally fused with the concretization norm
sum |y| * w and the gradient seed h = h_scale * sign(y) * w.  Shapes with
KH % sh == 0 and KW % sw == 0 run the parity-class MFMA kernel, the others the
row kernel; both are covered.  Tolerance: the fp32 accumulation bound
K * 2^-23 * sum |A| |W| of each output (K = contributing taps).
"""

import pytest
import torch
import torch.nn.functional as F

from boundflow_amd import _lib
from tests.gpu_util import announce, device

pytestmark = pytest.mark.gpu

# (R, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, S)
SHAPES = [
    (37, 32, 8, 8, 16, 4, 4, 2, 2, 1, 1, 9),     # C3 conv1 backward (MFMA path)
    (20, 16, 16, 16, 3, 4, 4, 2, 2, 1, 1, 4),    # C3 conv0 backward (MFMA path, Ci < 16)
    (9, 8, 7, 5, 20, 3, 3, 1, 1, 1, 1, 3),       # stride 1, 3x3, Ci > 16 (MFMA path, 9 taps)
    (6, 5, 6, 6, 4, 2, 2, 2, 2, 0, 0, 2),        # 2x2 stride 2, no padding (MFMA path)
    (7, 6, 5, 5, 3, 3, 3, 2, 2, 1, 1, 7),        # KH % sh != 0 (row kernel)
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
              KW, sh, sw, ph, pw, Hi, Wi, _lib.ptr(y_u), _lib.ptr(y_l), S, None, 0, None, None, None, None, st)
    # norm epilogue (Linf weights and box weights) with the gradient seed on the lower bound
    n_u = torch.empty(R, device=dev)
    n_l = torch.empty(R, device=dev)
    h = torch.empty(R, nout, device=dev)
    _lib.call("bf_conv_transpose_rows", _lib.ptr(Ad["u"]), _lib.ptr(Ad["l"]), R, Co, Ho, Wo, _lib.ptr(Wd), Ci, KH,
              KW, sh, sw, ph, pw, Hi, Wi, None, None, S, _lib.ptr(wvd), nout, _lib.ptr(n_u), _lib.ptr(n_l),
              _lib.ptr(hsd), _lib.ptr(h), st)
    n1 = torch.empty(R, device=dev)
    _lib.call("bf_conv_transpose_rows", None, _lib.ptr(Ad["l"]), R, Co, Ho, Wo, _lib.ptr(Wd), Ci, KH, KW, sh, sw, ph,
              pw, Hi, Wi, None, None, S, None, 0, None, _lib.ptr(n1), None, None, st)
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
