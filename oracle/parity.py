"""Parity judgement between the HIP path and the fp32 CPU oracle (test infrastructure only).

The contract is |hip - cpu32| <= 1e-6 + 1e-5 * |cpu32| for every bound.  Both
sides are fp32 computations of long sums with different summation orders, so
where a bound comes out of heavy cancellation (a margin near zero built from
terms of magnitude ~10) the two can differ by a few 1e-6 even though both are
correct fp32 results.  Such an element is accepted only when an fp64 run of
the same oracle shows that the HIP value is at least as close to the exact
value as the reference's own fp32 value is (within a factor of 2): the gap is
then the reference's rounding, not a HIP error.  Every such element is counted
and reported; any other mismatch fails.

Verdicts (certified = min over specs of the lower bound >= 0) must be
identical, except near-ties: rows whose reference minimum is within that
row's fp32 uncertainty of 0, which are counted and reported.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

RTOL = 1e-5
ATOL = 1e-6


@dataclass
class ParityReport:
    n: int
    max_abs: float
    max_rel: float
    strict_violations: int
    explained_by_fp32: int
    unexplained: int

    @property
    def ok(self) -> bool:
        return self.unexplained == 0

    def line(self, what: str) -> str:
        return (f"{what}: n={self.n} max_abs={self.max_abs:.3e} max_rel={self.max_rel:.3e} "
                f"strict_violations={self.strict_violations} (explained by fp32 cancellation: "
                f"{self.explained_by_fp32}, unexplained: {self.unexplained})")


def compare(got, ref32, ref64=None, rtol: float = RTOL, atol: float = ATOL) -> ParityReport:
    g = torch.as_tensor(got).detach().double().cpu()
    r = torch.as_tensor(ref32).detach().double().cpu()
    if g.shape != r.shape:
        raise AssertionError(f"shape {tuple(g.shape)} vs {tuple(r.shape)}")
    finite = torch.isfinite(r)
    d = (g - r).abs()
    d = torch.where(finite, d, torch.zeros_like(d))
    strict = (d > atol + rtol * r.abs()) & finite
    explained = torch.zeros_like(strict)
    if ref64 is not None and bool(strict.any()):
        e = torch.as_tensor(ref64).detach().double().cpu()
        err_hip = (g - e).abs()
        err_ref = (r - e).abs()
        explained = strict & (err_hip <= 2.0 * torch.maximum(err_ref, atol + rtol * e.abs()))
    rel = d / r.abs().clamp_min(1e-30)
    return ParityReport(
        n=int(finite.sum()),
        max_abs=float(d.max()) if d.numel() else 0.0,
        max_rel=float(rel[finite].max()) if bool(finite.any()) else 0.0,
        strict_violations=int(strict.sum()),
        explained_by_fp32=int(explained.sum()),
        unexplained=int((strict & ~explained).sum()),
    )


def verdicts(lower: torch.Tensor) -> torch.Tensor:
    return torch.as_tensor(lower).detach().cpu().min(dim=1).values >= 0


def verdict_parity(got_lower, ref32_lower, ref64_lower=None):
    """Return (mismatches, near_ties): rows whose certified flag differs, split
    into genuine mismatches and near-ties (reference minimum within its own
    fp32 uncertainty of zero)."""
    vg = verdicts(got_lower)
    vr = verdicts(ref32_lower)
    diff = vg != vr
    r = torch.as_tensor(ref32_lower).detach().double().cpu().min(dim=1).values
    unc = atol_row = ATOL + RTOL * r.abs()
    if ref64_lower is not None:
        e = torch.as_tensor(ref64_lower).detach().double().cpu().min(dim=1).values
        unc = torch.maximum(atol_row, 2.0 * (r - e).abs())
    tie = r.abs() <= unc
    return int((diff & ~tie).sum()), int((diff & tie).sum()), int(tie.sum())


def to_float64(w):
    """Copy of a workload (module params, spec, C) in float64 for the exact-value run."""
    from boundflow_amd import workloads as wl
    from boundflow_amd.ir import BFTaskModule
    from boundflow_amd.spec import BoxPerturbation, InputSpec

    params = {k: v.double() for k, v in w.module.params.items()}
    mod = BFTaskModule(tasks=w.module.tasks, entry_task_id=w.module.entry_task_id, bindings={"params": params},
                       storage_plan=w.module.storage_plan)
    p = w.spec.perturbation
    if isinstance(p, BoxPerturbation):
        spec = InputSpec.box(value_name=w.spec.value_name, lower=p.lower.double(), upper=p.upper.double())
    else:
        spec = InputSpec(value_name=w.spec.value_name, center=w.spec.center.double(), perturbation=p)
    return wl.Workload(w.name, mod, spec, w.C.double(), w.labels, dict(w.extra))
