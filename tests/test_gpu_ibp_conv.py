"""bf_ibp_conv2d through the C ABI against an fp64 restatement of interval propagation
through a conv layer (boundflow/domains/interval.py:57-86: center conv W, radius conv |W|;
the Linf ball input of boundflow/runtime/perturbation.py:102-173), with the consumer's ReLU
split applied as crown_ibp.py:70-98 does.  Covered: the one-launch kernel with its two
work splits (halves of the channel blocks, and pixel-tile parity, including a half with no
tile), box, ReLU-of-interval and ball inputs, and a layer whose two staged maps exceed the
one-launch kernel's LDS (the products-then-finalize path)."""

import pytest
import torch
import torch.nn.functional as F

from boundflow_amd import _lib
from tests.gpu_util import announce, device


def _reference(lo, hi, W, b, kind, eps, relu, split, stride, pad):
    W64 = W.double().cpu()
    if kind == 0:
        l, u = lo.double().cpu(), hi.double().cpu()
        if relu:
            l, u = l.clamp_min(0), u.clamp_min(0)
        mid, rad = (l + u) / 2, (u - l) / 2
    else:
        mid = lo.double().cpu()
        rad = torch.full_like(mid, eps)
    c = F.conv2d(mid, W64, stride=stride, padding=pad)
    dev = F.conv2d(rad, W64.abs(), stride=stride, padding=pad)
    mag = F.conv2d(mid.abs(), W64.abs(), stride=stride, padding=pad) + dev
    out_l, out_u = c - dev, c + dev
    if b is not None:
        bb = b.double().cpu().view(1, -1, 1, 1)
        out_l, out_u = out_l + bb, out_u + bb
    if split is not None:
        s = split.cpu().view_as(out_l)
        out_l = torch.where(s > 0, out_l.clamp_min(0), out_l)
        out_u = torch.where(s < 0, out_u.clamp_max(0), out_u)
    return out_l, out_u, c, mag


CASES = [
    # (B, Ci, H, Co, k, stride, pad, kind, relu, split)
    (5, 3, 32, 16, 4, 2, 1, 0, 0, True),    # C3's first conv, box input: one channel block, pixel-parity halves
    (4, 16, 16, 32, 4, 2, 1, 0, 1, True),   # C3's second conv on a ReLU interval: channel-block halves
    (3, 3, 32, 16, 4, 2, 1, 1, 0, False),   # Linf ball input
    (6, 5, 8, 24, 3, 1, 1, 0, 1, True),     # 24 channels: the second half's block is partly padding
    (2, 4, 6, 48, 3, 1, 0, 0, 1, False),    # three blocks, one pixel tile: the odd half has no task
    (2, 16, 20, 16, 3, 1, 1, 0, 1, True),   # two maps above the kernel's LDS: products, then finalize
]


@pytest.mark.gpu
@pytest.mark.parametrize("B,Ci,H,Co,k,stride,pad,kind,relu,with_split", CASES)
def test_ibp_conv2d_matches_fp64(B, Ci, H, Co, k, stride, pad, kind, relu, with_split):
    dev = device()
    announce(f"bf_ibp_conv2d B={B} Ci={Ci} H={H} Co={Co} k={k} s={stride} p={pad} kind={kind} relu={relu}")
    g = torch.Generator().manual_seed(B * 131 + Ci * 17 + H + Co)
    Ho = (H + 2 * pad - k) // stride + 1
    x = torch.randn(B, Ci, H, H, generator=g)
    w = torch.rand(B, Ci, H, H, generator=g) * 0.1
    lo = (x - w).to(dev)
    hi = (x + w).to(dev)
    W = (torch.randn(Co, Ci, k, k, generator=g) / (Ci * k * k) ** 0.5).to(dev)
    bias = (torch.randn(Co, generator=g) * 0.1).to(dev)
    eps = 0.03
    nin, nout = Ci * H * H, Co * Ho * Ho
    split = None
    if with_split:
        # two split neurons per domain, so that some domains are emptied and some are not
        s = torch.zeros(B, nout, dtype=torch.int8)
        rows = torch.arange(B).repeat_interleave(2)
        cols = torch.randint(0, nout, (2 * B,), generator=g)
        s[rows, cols] = (torch.randint(0, 2, (2 * B,), generator=g) * 2 - 1).to(torch.int8)
        split = s.to(dev)
    ws = torch.empty(int(_lib.load().bf_ibp_conv2d_workspace(B, nin, nout)), device=dev)
    out_l = torch.empty(B, Co, Ho, Ho, device=dev)
    out_u = torch.empty_like(out_l)
    cen = torch.empty_like(out_l)
    flags = torch.zeros(B, dtype=torch.int32, device=dev)
    _lib.call("bf_ibp_conv2d", _lib.ptr(lo), _lib.ptr(hi if kind == 0 else None), B, Ci, H, H, kind, eps, relu,
              _lib.ptr(W), _lib.ptr(bias), Co, k, k, stride, stride, pad, pad, Ho, Ho, _lib.ptr(split),
              nout if split is not None else 0, _lib.ptr(ws), _lib.ptr(out_l), _lib.ptr(out_u), _lib.ptr(cen),
              _lib.ptr(flags), _lib.stream_handle())
    torch.cuda.synchronize()
    ref_l, ref_u, ref_c, mag = _reference(lo, hi, W, bias, kind, eps, relu, split, stride, pad)
    tol = 2 * Ci * k * k * 2.0 ** -23 * mag + 1e-6
    for got, ref, what in ((out_l, ref_l, "lower"), (out_u, ref_u, "upper"), (cen, ref_c, "center")):
        err = (got.double().cpu() - ref).abs()
        bad = int((err > tol).sum())
        assert bad == 0, f"{what}: {bad} values outside the fp32 accumulation bound (max err {float(err.max()):.3g})"
    if split is not None:
        margin = (ref_l - ref_u).reshape(B, -1)
        t = tol.reshape(B, -1)
        clear = ~(margin.abs() <= t).any(1)
        want = (margin > 0).any(1).to(torch.int32)
        assert torch.equal(flags.cpu()[clear], want[clear])
    else:
        assert int(flags.sum()) == 0
