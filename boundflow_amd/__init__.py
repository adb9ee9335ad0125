"""boundflow_amd: MI355X-native (gfx950 HIP) bound-propagation hot path.

The package mirrors the reference's planner/runtime interfaces for the
IBP -> CROWN backward -> ReLU relaxation -> concretization -> alpha/beta
gradient path and runs every numeric step in hand-written HIP kernels
(``libboundflow_hip.so``, loaded through ctypes after torch).
"""

from .ir import BFTaskModule, BoundTask, BufferSpec, StoragePlan, TaskKind, TaskOp  # noqa: F401
from .spec import BoxPerturbation, InputSpec, IntervalState, LinfInputSpec, LpBallPerturbation  # noqa: F401

__all__ = [
    "BFTaskModule", "BoundTask", "BufferSpec", "StoragePlan", "TaskKind", "TaskOp",
    "BoxPerturbation", "InputSpec", "IntervalState", "LinfInputSpec", "LpBallPerturbation",
]
