"""bf_crown_relu_linear_concretize_noalloc (the concretization with its workspace in
a fixed device array) against bf_crown_relu_linear_concretize (caller workspace)
on the same inputs, through the C ABI: identical lower/upper bounds and
gradient seed on two calls in a row, the second smaller (the array keeps the
first call's contents), with Linf and box inputs; a size beyond the array is
refused before any launch."""

import pytest
import torch

from boundflow_amd import _lib
from tests.gpu_util import announce, device

pytestmark = pytest.mark.gpu


def _case(D, S, N, I, box, seed, dev):
    g = torch.Generator().manual_seed(seed)
    A_u = torch.randn(D, S, N, generator=g).to(dev)
    A_l = torch.randn(D, S, N, generator=g).to(dev)
    lo = (torch.randn(D, N, generator=g) - 0.3).to(dev)
    hi = lo + torch.rand(D, N, generator=g).to(dev)
    alpha = torch.rand(D, N, generator=g).to(dev)
    table = torch.empty(D, N, 4, device=dev)
    _lib.call("bf_relu_relax_table", _lib.ptr(lo), _lib.ptr(hi), _lib.ptr(alpha), N, D, N, _lib.ptr(table),
              _lib.stream_handle())
    add = (torch.randn(D, N, generator=g) * 0.1).to(dev)
    Wt = (torch.randn(I, N, generator=g) / N ** 0.5).to(dev)      # the layer weight transposed, [I, N]
    bias = torch.randn(N, generator=g).to(dev)
    cvec = torch.randn(D, N, generator=g).to(dev)
    rad = torch.rand(D, I, generator=g).to(dev) * 0.05 if box else None
    b_u = torch.randn(D * S, generator=g).to(dev)
    b_l = torch.randn(D * S, generator=g).to(dev)
    h_scale = torch.full((D * S,), -0.01, device=dev)
    return dict(A_u=A_u, A_l=A_l, table=table, add=add, Wt=Wt, bias=bias, cvec=cvec, rad=rad, eps=0.02, b_u=b_u,
                b_l=b_l, h_scale=h_scale, D=D, S=S, N=N, I=I)


def _run(c, noalloc):
    dev = c["A_u"].device
    D, S, N, I = c["D"], c["S"], c["N"], c["I"]
    lb = torch.full((D, S), float("nan"), device=dev)
    ub = torch.full((D, S), float("nan"), device=dev)
    h = torch.full((D * S, I), float("nan"), device=dev)
    args = [_lib.ptr(c["A_u"]), _lib.ptr(c["A_l"]), S * N, D, S, N, _lib.ptr(c["table"]), _lib.ptr(c["add"]), N,
            _lib.ptr(c["Wt"]), I, 1, _lib.ptr(c["bias"]), _lib.ptr(c["cvec"]), _lib.ptr(c["rad"]), c["eps"], 0,
            _lib.ptr(c["b_u"]), _lib.ptr(c["b_l"]), _lib.ptr(c["h_scale"]), _lib.ptr(h)]
    if noalloc:
        _lib.call("bf_crown_relu_linear_concretize_noalloc", *args, _lib.ptr(lb), _lib.ptr(ub), _lib.stream_handle())
    else:
        ws = torch.empty(int(_lib.load().bf_crown_relu_linear_concretize_workspace(D, S, I)), device=dev)
        _lib.call("bf_crown_relu_linear_concretize", *args, _lib.ptr(ws), _lib.ptr(lb), _lib.ptr(ub),
                  _lib.stream_handle())
    torch.cuda.synchronize()
    return lb, ub, h


@pytest.mark.parametrize("box", [False, True])
def test_noalloc_matches_workspace_entry_point(box):
    dev = device()
    for call, (D, S, N, I) in enumerate([(64, 9, 256, 784), (16, 9, 100, 300)]):
        announce(f"concretize noalloc vs workspace, call {call}: D={D} S={S} N={N} I={I} box={box}")
        c = _case(D, S, N, I, box, 7 + call, dev)
        ref = _run(c, noalloc=False)
        got = _run(c, noalloc=True)
        for name, r, x in zip(("lower", "upper", "gradient seed"), ref, got):
            assert torch.isfinite(x).all(), f"call {call}: {name} has unwritten elements"
            assert torch.equal(x, r), f"call {call}: {name} differs"


def test_noalloc_refuses_sizes_beyond_its_array():
    dev = device()
    announce("concretize noalloc: size beyond the fixed array is refused")
    D, S, N, I = 30000, 9, 16, 784    # (2 * 7 + 4) * 270000 floats > 4M
    dummy = torch.zeros(4, device=dev)
    rc = _lib.load().bf_crown_relu_linear_concretize_noalloc(
        _lib.ptr(dummy), None, S * N, D, S, N, None, None, 0, _lib.ptr(dummy), I, 1, None, _lib.ptr(dummy), None,
        0.01, 0, None, None, None, None, None, _lib.ptr(dummy), _lib.stream_handle())
    assert rc == 3
    assert b"fixed scratch" in _lib.load().bf_last_error()
