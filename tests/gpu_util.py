"""Shared helpers for the HIP parity tests."""

import sys

import pytest
import torch

# Bound tolerance of the parity contract: |hip - ref| <= ATOL + RTOL * |ref|
RTOL = 1e-5
ATOL = 1e-6


def device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from boundflow_amd import _lib
    _lib.load()  # raise loudly if the library is missing
    return torch.device("cuda:0")


def announce(msg: str) -> None:
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


def err_report(got: torch.Tensor, ref: torch.Tensor):
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    d = (g - r).abs()
    rel = d / r.abs().clamp_min(1e-30)
    viol = d > (ATOL + RTOL * r.abs())
    return float(d.max()) if d.numel() else 0.0, float(rel.max()) if rel.numel() else 0.0, int(viol.sum())


def assert_bounds_close(got: torch.Tensor, ref: torch.Tensor, what: str, rtol: float = RTOL, atol: float = ATOL):
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    assert g.shape == r.shape, f"{what}: shape {tuple(g.shape)} vs {tuple(r.shape)}"
    d = (g - r).abs()
    bad = d > (atol + rtol * r.abs())
    amax = float(d.max()) if d.numel() else 0.0
    announce(f"{what}: max abs err {amax:.3e}, violations {int(bad.sum())}/{d.numel()}")
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} elements outside rtol={rtol} atol={atol} (max abs {amax})"


def contraction_tol(a: torch.Tensor, b: torch.Tensor, k: int) -> torch.Tensor:
    """fp32 accumulation error bound for C = a @ b: k * 2^-23 * (|a| @ |b|)."""
    return k * (2.0 ** -23) * (a.abs().double() @ b.abs().double())


def assert_parity(got, ref32, ref64, what: str):
    """Contract tolerance, with fp32-cancellation mismatches accepted only when
    the fp64 oracle shows the HIP value is as close to exact as the reference."""
    from oracle import parity
    rep = parity.compare(got, ref32, ref64)
    announce(rep.line(what))
    assert rep.ok, rep.line(what)
    return rep


def assert_verdicts(got_lower, ref32_lower, ref64_lower, what: str):
    from oracle import parity
    mism, ties_flipped, ties = parity.verdict_parity(got_lower, ref32_lower, ref64_lower)
    announce(f"{what}: verdict mismatches={mism} near-tie flips={ties_flipped} near-ties={ties}")
    assert mism == 0, f"{what}: {mism} verdict mismatches"
