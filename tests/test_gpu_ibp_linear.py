"""bf_ibp_linear through the C ABI against an fp64 restatement of interval propagation
through a linear layer (boundflow/domains/interval.py:57-86 for intervals,
boundflow/runtime/perturbation.py:102-173 for the input balls), with the consumer's ReLU
split applied as crown_ibp.py:70-98 does.  Small outputs take the one-launch kernel
(products and finalize in one workgroup per 16 x 16 tile); larger ones the split-K
contraction and the finalize kernel: both routes are covered, on ragged sizes, unaligned
reduction lengths and reductions longer than one round of loads."""

import pytest
import torch

from boundflow_amd import _lib
from tests.gpu_util import announce, device


def _reference(lo, hi, W, b, kind, eps, relu, split):
    lo64, W64 = lo.double().cpu(), W.double().cpu()
    if kind == 0:
        l, u = lo64, hi.double().cpu()
        if relu:
            l, u = l.clamp_min(0), u.clamp_min(0)
        mid, rad = (l + u) / 2, (u - l) / 2
        c = mid @ W64.t()
        dev = rad @ W64.abs().t()
        mag = mid.abs() @ W64.abs().t() + dev
    else:
        c = lo64 @ W64.t()
        norm = {1: W64.abs().sum(1), 2: W64.pow(2).sum(1).sqrt(), 3: W64.abs().amax(1)}[kind]
        dev = (eps * norm).expand_as(c)
        mag = lo64.abs() @ W64.abs().t() + dev
    out_l, out_u = c - dev, c + dev
    if b is not None:
        out_l, out_u = out_l + b.double().cpu(), out_u + b.double().cpu()
    if split is not None:
        s = split.cpu()
        out_l = torch.where(s > 0, out_l.clamp_min(0), out_l)
        out_u = torch.where(s < 0, out_u.clamp_max(0), out_u)
    return out_l, out_u, c, mag


def _run(lo, hi, W, b, kind, eps, relu, split, want_center):
    B, K = lo.shape
    N = W.shape[0]
    dev = lo.device
    ws = torch.empty(max(1, int(_lib.load().bf_ibp_linear_workspace(B, K, N))), device=dev)
    out_l = torch.empty(B, N, device=dev)
    out_u = torch.empty(B, N, device=dev)
    cen = torch.empty(B, N, device=dev) if want_center else None
    flags = torch.zeros(B, dtype=torch.int32, device=dev)
    _lib.call("bf_ibp_linear", _lib.ptr(lo), _lib.ptr(hi), B, K, kind, eps, relu, _lib.ptr(W), _lib.ptr(b), N,
              _lib.ptr(split), N if split is not None else 0, _lib.ptr(ws), _lib.ptr(out_l), _lib.ptr(out_u),
              _lib.ptr(cen), _lib.ptr(flags), None, _lib.stream_handle())
    torch.cuda.synchronize()
    return out_l, out_u, cen, flags


CASES = [
    # (B, K, N, kind, relu, with split): kind 0 interval, 1 Linf ball, 2 L2 ball, 3 L1 ball
    (37, 301, 45, 0, 1, True),      # ragged, K % 4 != 0 (scalar loads)
    (64, 784, 256, 0, 0, False),    # a box input layer of C1's shape
    (128, 2048, 100, 0, 1, True),   # more k steps than one round of loads
    (5, 200, 33, 1, 0, False),
    (5, 200, 33, 2, 0, True),
    (5, 203, 33, 3, 0, False),
    (1, 3072, 17, 0, 1, False),     # one row, long reduction
    (512, 96, 600, 0, 1, True),     # 1216 tiles of 16 x 16: the split-K contraction route
    (300, 500, 500, 1, 0, False),   # a ball on the contraction route
]


@pytest.mark.gpu
@pytest.mark.parametrize("B,K,N,kind,relu,with_split", CASES)
def test_ibp_linear_matches_fp64(B, K, N, kind, relu, with_split):
    dev = device()
    announce(f"bf_ibp_linear B={B} K={K} N={N} kind={kind} relu={relu} split={with_split}")
    g = torch.Generator().manual_seed(B * 7919 + K * 31 + N)
    x = torch.randn(B, K, generator=g)
    w = torch.rand(B, K, generator=g) * (2.0 / K ** 0.5)   # narrow enough that many neurons are stable
    lo = (x - w).to(dev)
    hi = (x + w).to(dev) if kind == 0 else lo
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(dev)
    b = (torch.randn(N, generator=g) * 0.1).to(dev)
    eps = 0.05
    split = None
    if with_split:
        # two split neurons per domain, so that some domains are emptied and some are not
        split = torch.zeros(B, N, dtype=torch.int8)
        rows = torch.arange(B).repeat_interleave(2)
        cols = torch.randint(0, N, (2 * B,), generator=g)
        split[rows, cols] = (torch.randint(0, 2, (2 * B,), generator=g) * 2 - 1).to(torch.int8)
        split = split.to(dev)
    ref_l, ref_u, ref_c, mag = _reference(lo, hi, W, b, kind, eps, relu, split)
    got_l, got_u, got_c, flags = _run(lo, hi, W, b, kind, eps, relu, split, want_center=True)
    tol = 2 * K * 2.0 ** -23 * mag + 1e-6
    for got, ref, what in ((got_l, ref_l, "lower"), (got_u, ref_u, "upper"), (got_c, ref_c, "center")):
        err = (got.double().cpu() - ref).abs()
        bad = int((err > tol).sum())
        assert bad == 0, f"{what}: {bad} values outside the fp32 accumulation bound (max err {float(err.max()):.3g})"
    if split is not None:
        # a domain's flag is set when a split empties a box; domains with a box within
        # rounding of empty are left out
        margin = ref_l - ref_u
        clear = ~(margin.abs() <= tol).any(1)
        want = (margin > 0).any(1).to(torch.int32)
        assert torch.equal(flags.cpu()[clear], want[clear])
        assert int(want[clear].sum()) > 0, "the split cases must flag some domain"
        if int(clear.sum()) >= 10:
            assert int(want[clear].sum()) < int(clear.sum()), "and leave some domain unflagged"
    else:
        assert int(flags.sum()) == 0


@pytest.mark.gpu
def test_ibp_linear_without_center_output_or_bias():
    """center_out, bias and split may each be NULL; the bounds do not change with center_out."""
    dev = device()
    g = torch.Generator().manual_seed(11)
    B, K, N = 20, 130, 40
    x = torch.randn(B, K, generator=g)
    lo = (x - 0.1).to(dev)
    hi = (x + 0.1).to(dev)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(dev)
    a_l, a_u, _, _ = _run(lo, hi, W, None, 0, 0.0, 1, None, want_center=False)
    b_l, b_u, _, _ = _run(lo, hi, W, None, 0, 0.0, 1, None, want_center=True)
    assert torch.equal(a_l, b_l) and torch.equal(a_u, b_u)
    ref_l, ref_u, _, mag = _reference(lo, hi, W, None, 0, 0.0, 1, None)
    tol = 2 * K * 2.0 ** -23 * mag + 1e-6
    assert bool(((a_l.double().cpu() - ref_l).abs() <= tol).all())
    assert bool(((a_u.double().cpu() - ref_u).abs() <= tol).all())


@pytest.mark.gpu
@pytest.mark.parametrize("B,K,N", [(64, 784, 256), (37, 301, 45), (512, 96, 600)])
def test_ibp_linear_box_radius_output(B, K, N):
    """box_radius_out receives (hi - lo) / 2 of the input box, bit for bit as torch's fp32
    arithmetic makes it, on the one-launch route (written from the loaded bounds, including
    K % 4 != 0) and on the split-K contraction route (its own launch); the bounds are the
    same as without it."""
    dev = device()
    g = torch.Generator().manual_seed(B + K + N)
    x = torch.randn(B, K, generator=g)
    w = torch.rand(B, K, generator=g)
    lo = (x - w).to(dev)
    hi = (x + w).to(dev)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(dev)
    ws = torch.empty(max(1, int(_lib.load().bf_ibp_linear_workspace(B, K, N))), device=dev)
    outs = []
    for with_rad in (False, True):
        out_l = torch.empty(B, N, device=dev)
        out_u = torch.empty(B, N, device=dev)
        rad = torch.full((B, K), float("nan"), device=dev) if with_rad else None
        _lib.call("bf_ibp_linear", _lib.ptr(lo), _lib.ptr(hi), B, K, 0, 0.0, 0, _lib.ptr(W), None, N, None, 0,
                  _lib.ptr(ws), _lib.ptr(out_l), _lib.ptr(out_u), None, None, _lib.ptr(rad), _lib.stream_handle())
        outs.append((out_l, out_u, rad))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[1][2], (hi - lo) / 2)


@pytest.mark.gpu
def test_ibp_linear_box_radius_refuses_relu_or_ball():
    dev = device()
    lo = torch.zeros(2, 8, device=dev)
    W = torch.ones(3, 8, device=dev)
    ws = torch.empty(int(_lib.load().bf_ibp_linear_workspace(2, 8, 3)), device=dev)
    out = torch.empty(2, 3, device=dev)
    rad = torch.empty(2, 8, device=dev)
    for kind, relu in ((0, 1), (1, 0)):
        with pytest.raises(_lib.HipError, match="box_radius_out"):
            _lib.call("bf_ibp_linear", _lib.ptr(lo), _lib.ptr(lo), 2, 8, kind, 0.1, relu, _lib.ptr(W), None, 3, None,
                      0, _lib.ptr(ws), _lib.ptr(out), _lib.ptr(out), None, None, _lib.ptr(rad),
                      _lib.stream_handle())
