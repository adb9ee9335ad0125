"""Bound/perturbation data types shared by the HIP backend and its callers.

Mirrors of the reference's data contracts (no computation lives here):

* ``IntervalState`` -- boundflow/domains/interval.py:13-24
* ``LpBallPerturbation`` -- boundflow/runtime/perturbation.py:73-104
* ``BoxPerturbation`` -- boundflow/runtime/perturbation.py:225-261
* ``InputSpec`` / ``LinfInputSpec`` -- boundflow/runtime/task_executor.py:24-74
* ``normalize_input_spec`` -- boundflow/runtime/task_executor.py:566-571
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Union

import torch


@dataclass
class IntervalState:
    lower: torch.Tensor
    upper: torch.Tensor

    def validate(self) -> None:
        if self.lower.shape != self.upper.shape:
            raise ValueError(f"interval shape mismatch: {self.lower.shape} vs {self.upper.shape}")
        if self.lower.dtype != self.upper.dtype:
            raise ValueError(f"interval dtype mismatch: {self.lower.dtype} vs {self.upper.dtype}")
        if self.lower.device != self.upper.device:
            raise ValueError(f"interval device mismatch: {self.lower.device} vs {self.upper.device}")


@dataclass(frozen=True)
class LpBallPerturbation:
    """Lp ball of radius ``eps`` around the center; p in {inf, 1, 2}."""

    p: Union[str, float, int]
    eps: float

    def normalized_p(self) -> str:
        p = self.p
        if isinstance(p, str):
            s = p.strip().lower()
            if s in {"inf", "l_inf", "linf"}:
                return "inf"
            raise ValueError(f"unsupported p string for LpBallPerturbation: {self.p!r}")
        if int(p) == p and int(p) in (1, 2):
            return str(int(p))
        if float(p) == float("inf"):
            return "inf"
        raise ValueError(f"unsupported p for LpBallPerturbation: {self.p!r}")

    @property
    def perturbation_id(self) -> str:
        return f"lp(p={self.normalized_p()},eps={float(self.eps)})"

    def bounding_box(self, center: torch.Tensor):
        eps = float(self.eps)
        return center - eps, center + eps


@dataclass(frozen=True)
class BoxPerturbation:
    """Per-element input box (clipped Linf balls, VNNLIB boxes)."""

    lower: torch.Tensor
    upper: torch.Tensor

    def __post_init__(self) -> None:
        if not torch.is_tensor(self.lower) or not torch.is_tensor(self.upper):
            raise TypeError("BoxPerturbation bounds must be torch tensors")
        if self.lower.shape != self.upper.shape:
            raise ValueError(
                f"BoxPerturbation shape mismatch: lower={tuple(self.lower.shape)} upper={tuple(self.upper.shape)}"
            )
        if self.lower.device != self.upper.device or self.lower.dtype != self.upper.dtype:
            raise ValueError("BoxPerturbation bounds must share device and dtype")
        if not torch.is_floating_point(self.lower):
            raise TypeError("BoxPerturbation bounds must be floating point")
        if not bool(torch.isfinite(self.lower).all() and torch.isfinite(self.upper).all()):
            raise ValueError("BoxPerturbation bounds must be finite")
        if not bool((self.lower <= self.upper).all()):
            raise ValueError("BoxPerturbation requires lower <= upper")
        object.__setattr__(self, "lower", self.lower.detach().clone())
        object.__setattr__(self, "upper", self.upper.detach().clone())

    def bounding_box(self, center: torch.Tensor):
        return self.lower, self.upper


@dataclass(frozen=True)
class LinfInputSpec:
    value_name: str
    center: torch.Tensor
    eps: float


def input_norm_p(pert) -> int:
    """Norm code of the input concretization (perturbation.py:175-222): 0 for a Linf ball
    or a box (sum |A|, radius-weighted for a box), 1 for an L1 ball (its dual norm
    max |A|), 2 for an L2 ball (the row's L2 norm)."""
    if isinstance(pert, BoxPerturbation):
        return 0
    return {"inf": 0, "1": 1, "2": 2}[pert.normalized_p()]


@dataclass(frozen=True)
class InputSpec:
    value_name: str
    center: torch.Tensor
    perturbation: Union[LpBallPerturbation, BoxPerturbation]

    @staticmethod
    def linf(*, value_name: str, center: torch.Tensor, eps: float) -> "InputSpec":
        return InputSpec(value_name=value_name, center=center, perturbation=LpBallPerturbation(p="inf", eps=eps))

    @staticmethod
    def l2(*, value_name: str, center: torch.Tensor, eps: float) -> "InputSpec":
        return InputSpec(value_name=value_name, center=center, perturbation=LpBallPerturbation(p=2, eps=eps))

    @staticmethod
    def l1(*, value_name: str, center: torch.Tensor, eps: float) -> "InputSpec":
        return InputSpec(value_name=value_name, center=center, perturbation=LpBallPerturbation(p=1, eps=eps))

    @staticmethod
    def box(*, value_name: str, lower: torch.Tensor, upper: torch.Tensor) -> "InputSpec":
        return InputSpec(
            value_name=value_name,
            center=(lower + upper) / 2.0,
            perturbation=BoxPerturbation(lower=lower, upper=upper),
        )

    def to(self, device) -> "InputSpec":
        """Same specification with every tensor moved to ``device``."""
        p = self.perturbation
        if isinstance(p, BoxPerturbation):
            p = BoxPerturbation(lower=p.lower.to(device), upper=p.upper.to(device))
        return InputSpec(value_name=self.value_name, center=self.center.to(device), perturbation=p)


InputSpecLike = Union[LinfInputSpec, InputSpec]


def normalize_input_spec(spec: InputSpecLike) -> InputSpec:
    if isinstance(spec, InputSpec):
        return spec
    return InputSpec.linf(value_name=spec.value_name, center=spec.center, eps=float(spec.eps))
