"""Fused ReLU->Affine CROWN region contract and its HIP executor.

The dataclasses and planning helpers carry the reference's backend-neutral
contract unchanged (boundflow/runtime/fused_crown.py):

* ``FusedReluAffineRequest`` / ``FusedReluAffineResult``      -- :33-58
* ``FusedCrownExecutionContext``                              -- :61-69
* ``FusedCrownExecutionStep``, ``FusedCrownRuntimeSelection`` -- :72-94
* ``FusedCrownExecutor`` protocol                             -- :97-123
* ``FusedReluAffineDescriptor``                               -- :137-149
* ``fused_crown_graph_fingerprint``                           -- :152-168
* ``plan_fused_crown_regions`` / ``validate_fused_crown_execution_steps`` -- :178-276
* ``build_fused_crown_runtime_selection``                     -- :826-847
* ``HipTaskBackendRegistry``: the typed-registry entry of the HIP backend, the
  counterpart of ``TVMTaskBackendRegistry.dispatch``
  (boundflow/runtime/task_backend_dispatch.py:421-495) after its key validation

with one addition: the backend id ``"hip_fused"`` in the step whitelist and the
runtime selection, mapped to ``HipFusedCrownExecutor``.  That executor accepts
every plain-CROWN fp32 linear region and conv2d regions with groups 1 /
dilation 1 (any kernel size, stride and padding -- the reference's TVM kernel
rejects the 4x4 kernels of the benchmark CNN) and runs them on the caller's
stream through the C ABI; it allocates the four outputs with the torch
allocator, as the reference executors do (fused_crown.py:704-718).
"""

from __future__ import annotations

import contextlib
import hashlib
import json
from dataclasses import dataclass
from enum import Enum
from typing import Any, Literal, Mapping, Optional, Protocol, Sequence, Tuple

import torch

from . import _lib
from .conv import packed_conv_transpose_weights
from .crown import EPILOGUE_MIN_M, RELAX_PASS_MIN_K, derived, transposed
from .profiling import launch as _timed


class BoundaryRepresentation(Enum):
    DENSE = "dense"
    STRUCTURED = "structured"


class InternalMaterializationPolicy(Enum):
    EAGER = "eager"
    ELIDE_RELU_SCALED_A = "elide_relu_scaled_a"


@dataclass(frozen=True)
class FusedReluAffineRequest:
    kind: Literal["linear", "conv2d"]
    A_u: torch.Tensor
    A_l: torch.Tensor
    alpha_u: torch.Tensor
    alpha_l: torch.Tensor
    beta_u: torch.Tensor
    beta_l: torch.Tensor
    weight: torch.Tensor
    bias: Optional[torch.Tensor]
    input_shape: Tuple[int, ...]
    output_shape: Tuple[int, ...]
    attrs: Mapping[str, object]


@dataclass(frozen=True)
class FusedReluAffineResult:
    A_prev_u: torch.Tensor
    A_prev_l: torch.Tensor
    bias_delta_u: torch.Tensor
    bias_delta_l: torch.Tensor


@dataclass(frozen=True)
class FusedCrownExecutionContext:
    plain_crown: bool = True
    requires_grad: bool = False
    alpha_enabled: bool = False
    beta_enabled: bool = False
    split_state_present: bool = False


@dataclass(frozen=True)
class FusedCrownExecutionStep:
    kind: Literal["fused_relu_linear", "fused_relu_conv2d"]
    relu_op_index: int
    affine_op_index: int
    consumed_outputs: Tuple[str, str]
    graph_fingerprint: str
    boundary_representation: BoundaryRepresentation = BoundaryRepresentation.DENSE
    internal_materialization: InternalMaterializationPolicy = InternalMaterializationPolicy.ELIDE_RELU_SCALED_A
    backend: str = "tvm_fused_tir"


@dataclass(frozen=True)
class FusedCrownRuntimeSelection:
    backend: str
    executor: Optional["FusedCrownExecutor"]
    steps: Tuple[FusedCrownExecutionStep, ...]


@dataclass(frozen=True)
class FusedReluAffineDescriptor:
    kind: Literal["linear", "conv2d"]
    coefficient_shape: Tuple[int, int, int]
    weight: torch.Tensor
    bias: Optional[torch.Tensor]
    input_shape: Tuple[int, ...]
    output_shape: Tuple[int, ...]
    attrs: Mapping[str, object]
    device: torch.device
    dtype: torch.dtype


class FusedCrownExecutor(Protocol):
    def supports_descriptor(self, descriptor: FusedReluAffineDescriptor,
                            context: FusedCrownExecutionContext) -> bool: ...

    def supports(self, request: FusedReluAffineRequest, context: FusedCrownExecutionContext) -> bool: ...

    def run(self, request: FusedReluAffineRequest, *,
            stream: Optional[torch.cuda.Stream] = None) -> FusedReluAffineResult: ...


_BACKENDS = {"tvm_fused_tir", "tvm_tir_unfused", "pytorch_chunked", "hip_fused"}


def fused_crown_graph_fingerprint(ops: Sequence[Any]) -> str:
    payload = [
        {
            "index": index,
            "op_type": op.op_type,
            "name": op.name,
            "inputs": list(op.inputs),
            "outputs": list(op.outputs),
            "attrs": sorted((str(key), repr(value)) for key, value in op.attrs.items()),
        }
        for index, op in enumerate(ops)
    ]
    encoded = json.dumps(payload, sort_keys=True, separators=(",", ":")).encode()
    return hashlib.sha256(encoded).hexdigest()


def _consumers(ops: Sequence[Any]):
    out: dict = {}
    for index, op in enumerate(ops):
        for name in op.inputs:
            out.setdefault(name, []).append(index)
    return {k: tuple(v) for k, v in out.items()}


def plan_fused_crown_regions(ops: Sequence[Any], *, backend: str = "hip_fused") -> Tuple[FusedCrownExecutionStep, ...]:
    """Match forward Affine->ReLU pairs whose affine output feeds only the ReLU."""
    if backend not in _BACKENDS:
        raise ValueError(f"unsupported fused CROWN backend: {backend}")
    steps = []
    consumers = _consumers(ops)
    fp = fused_crown_graph_fingerprint(ops)
    for relu_index, relu_op in enumerate(ops):
        if relu_op.op_type != "relu" or relu_index == 0:
            continue
        affine = ops[relu_index - 1]
        if affine.op_type not in {"linear", "conv2d"}:
            continue
        if len(affine.outputs) != 1 or tuple(relu_op.inputs) != tuple(affine.outputs):
            continue
        if consumers.get(affine.outputs[0], ()) != (relu_index,):
            continue
        kind = "fused_relu_linear" if affine.op_type == "linear" else "fused_relu_conv2d"
        steps.append(FusedCrownExecutionStep(kind=kind, relu_op_index=relu_index, affine_op_index=relu_index - 1,
                                             consumed_outputs=(relu_op.outputs[0], affine.outputs[0]),
                                             graph_fingerprint=fp, backend=backend))
    return tuple(steps)


def validate_fused_crown_execution_steps(ops: Sequence[Any],
                                         steps: Sequence[FusedCrownExecutionStep]) -> Tuple[FusedCrownExecutionStep, ...]:
    """Keep only graph-current, single-consumer, supported steps."""
    fp = fused_crown_graph_fingerprint(ops)
    consumers = _consumers(ops)
    valid = []
    seen_relu: set = set()
    seen_affine: set = set()
    for step in steps:
        if step.graph_fingerprint != fp:
            continue
        if step.relu_op_index in seen_relu or step.affine_op_index in seen_affine:
            continue
        if not 0 <= step.affine_op_index < step.relu_op_index < len(ops):
            continue
        if step.relu_op_index != step.affine_op_index + 1:
            continue
        affine = ops[step.affine_op_index]
        relu = ops[step.relu_op_index]
        expected = "fused_relu_linear" if affine.op_type == "linear" else "fused_relu_conv2d"
        if affine.op_type not in {"linear", "conv2d"} or step.kind != expected:
            continue
        if relu.op_type != "relu" or tuple(relu.inputs) != tuple(affine.outputs):
            continue
        if len(affine.outputs) != 1 or len(relu.outputs) != 1:
            continue
        if step.consumed_outputs != (relu.outputs[0], affine.outputs[0]):
            continue
        if consumers.get(affine.outputs[0], ()) != (step.relu_op_index,):
            continue
        if step.boundary_representation != BoundaryRepresentation.DENSE:
            continue
        if step.internal_materialization != InternalMaterializationPolicy.ELIDE_RELU_SCALED_A:
            continue
        if step.backend not in _BACKENDS:
            continue
        valid.append(step)
        seen_relu.add(step.relu_op_index)
        seen_affine.add(step.affine_op_index)
    return tuple(valid)


def _pair(attrs: Mapping[str, object], name: str, default: Tuple[int, int]) -> Tuple[int, int]:
    v = attrs.get(name, default)
    if isinstance(v, int):
        return (v, v)
    if isinstance(v, (list, tuple)) and len(v) == 2:
        return (int(v[0]), int(v[1]))
    raise ValueError(f"{name} expects an integer pair, got {v!r}")


class HipFusedCrownExecutor:
    """FusedCrownExecutor backed by libboundflow_hip (backend id "hip_fused")."""

    def supports_descriptor(self, descriptor: FusedReluAffineDescriptor,
                            context: FusedCrownExecutionContext) -> bool:
        if not (context.plain_crown and not context.requires_grad and not context.alpha_enabled
                and not context.beta_enabled and not context.split_state_present):
            return False
        if descriptor.dtype != torch.float32 or descriptor.device.type != "cuda":
            return False
        if descriptor.kind == "linear":
            return descriptor.weight.dim() == 2
        if descriptor.kind == "conv2d":
            a = descriptor.attrs
            if int(a.get("groups", 1)) != 1 or _pair(a, "dilation", (1, 1)) != (1, 1):
                return False
            return descriptor.weight.dim() == 4
        return False

    def supports(self, request: FusedReluAffineRequest, context: FusedCrownExecutionContext) -> bool:
        tensors = [request.A_u, request.A_l, request.alpha_u, request.alpha_l, request.beta_u, request.beta_l,
                   request.weight] + ([request.bias] if request.bias is not None else [])
        return bool(context.plain_crown and not context.requires_grad and not context.alpha_enabled
                    and not context.beta_enabled and not context.split_state_present
                    and request.kind in ("linear", "conv2d")
                    and all(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous() and not t.requires_grad
                            for t in tensors))

    def run(self, request: FusedReluAffineRequest, *,
            stream: Optional[torch.cuda.Stream] = None) -> FusedReluAffineResult:
        # every launch, and the torch ops that prepare operands, go to the caller's stream
        with (torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()):
            return self._run(request, _lib.stream_handle(stream))

    def _run(self, request: FusedReluAffineRequest, st) -> FusedReluAffineResult:
        """A linear region: the four relaxation tensors interleaved into the kernels' table
        (one small launch), then the fused relaxation + contraction (a region of few rows:
        the relaxation pass, then the plain contraction).  A conv region: one
        launch, the channel-last transposed convolution reading the four tensors while it
        stages each row; conv shapes that kernel does not take run the relaxation pass and
        then the transposed convolution."""
        dev = request.A_u.device
        D, S = int(request.A_u.shape[0]), int(request.A_u.shape[1])
        M = D * S
        N = int(request.alpha_u.reshape(D, -1).shape[1])
        planes = [request.alpha_u, request.beta_u, request.alpha_l, request.beta_l]
        bias = None if request.bias is None else request.bias.contiguous()
        du = torch.empty(D, S, device=dev, dtype=torch.float32)
        dl = torch.empty(D, S, device=dev, dtype=torch.float32)
        if request.kind == "linear":
            P = int(request.weight.shape[1])
            Wt = transposed(request.weight)   # [P, N]: the kernel's faster operand layout, kept across calls
            pu = torch.empty(D, S, P, device=dev, dtype=torch.float32)
            pl = torch.empty(D, S, P, device=dev, dtype=torch.float32)
            table = torch.empty(D * N * 4, device=dev, dtype=torch.float32)
            with _timed("executor_relax_table", 0.0, 4.0 * 8 * D * N):
                _lib.call("bf_relu_relax_table_from_planes", *[_lib.ptr(t) for t in planes], D * N, _lib.ptr(table), st)
            if M < EPILOGUE_MIN_M and N >= RELAX_PASS_MIN_K:
                # a region of few rows: the relaxation pass, then the plain-prologue contraction,
                # whose 64 x 64 tiles spread the short grid over more CUs (as crown_backward does)
                ru = torch.empty(M, N, device=dev, dtype=torch.float32)
                rl = torch.empty(M, N, device=dev, dtype=torch.float32)
                with _timed("executor_relu_relax", 0.0, 4.0 * (4 * M * N + 4 * D * N)):
                    _lib.call("bf_crown_relu_relax", _lib.ptr(request.A_u), _lib.ptr(request.A_l), S * N, D, S, N,
                              _lib.ptr(table), None, 0, _lib.ptr(bias), None, None, None, _lib.ptr(ru), _lib.ptr(rl),
                              _lib.ptr(du), _lib.ptr(dl), None, None, st)
                with _timed("executor_linear", 4.0 * M * N * P, 4.0 * (2 * M * N + N * P + 2 * M * P)):
                    _lib.call("bf_crown_relu_linear_fwd", _lib.ptr(ru), _lib.ptr(rl), S * N, D, S, N, None, None, 0,
                              _lib.ptr(Wt), P, 1, None, None, None, _lib.ptr(pu), _lib.ptr(pl), None, None, st)
                return FusedReluAffineResult(pu, pl, du, dl)
            with _timed("executor_relu_linear", 4.0 * M * N * P, 4.0 * (2 * M * N + 4 * D * N + N * P + 2 * M * P)):
                _lib.call("bf_crown_relu_linear_fwd", _lib.ptr(request.A_u), _lib.ptr(request.A_l), S * N, D, S, N,
                          _lib.ptr(table), None, 0, _lib.ptr(Wt), P, 1, _lib.ptr(bias), None, None, _lib.ptr(pu),
                          _lib.ptr(pl), _lib.ptr(du), _lib.ptr(dl), st)
            return FusedReluAffineResult(pu, pl, du, dl)
        Co, Ho, Wo = (int(d) for d in request.output_shape)
        Ci, Hi, Wi = (int(d) for d in request.input_shape)
        W = request.weight.contiguous()
        KH, KW = int(W.shape[2]), int(W.shape[3])
        sh, sw = _pair(request.attrs, "stride", (1, 1))
        ph, pw = _pair(request.attrs, "padding", (0, 0))
        kbias = None if bias is None else derived(
            f"conv_bias_map:{Ho}x{Wo}", (bias,), lambda: bias.reshape(Co, 1).expand(Co, Ho * Wo).reshape(-1).contiguous())
        pu = torch.empty(D, S, Ci, Hi, Wi, device=dev)
        pl = torch.empty(D, S, Ci, Hi, Wi, device=dev)
        flops = 4.0 * M * Co * Ho * Wo * Ci * KH * KW / (sh * sw)
        if _lib.load().bf_conv_transpose_hwc_supported(Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi):
            wpk = packed_conv_transpose_weights(W, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi)
            with _timed("executor_relu_conv_transpose", flops, 4.0 * (2 * M * N + 4 * D * N + 2 * M * Ci * Hi * Wi)):
                _lib.call("bf_crown_relu_planes_conv_transpose", _lib.ptr(request.A_u), _lib.ptr(request.A_l), D, S,
                          Co, Ho, Wo, *[_lib.ptr(t) for t in planes], _lib.ptr(kbias), None, None, _lib.ptr(W),
                          _lib.ptr(wpk), Ci, KH, KW, sh, sw, ph, pw, Hi, Wi, _lib.ptr(pu), _lib.ptr(pl),
                          _lib.ptr(du), _lib.ptr(dl), st)
            return FusedReluAffineResult(pu, pl, du, dl)
        # other conv shapes: the relaxation pass (from the interleaved table), then the transposed convolution
        table = torch.empty(D * N * 4, device=dev, dtype=torch.float32)
        _lib.call("bf_relu_relax_table_from_planes", *[_lib.ptr(t) for t in planes], D * N, _lib.ptr(table), st)
        ru = torch.empty(M, N, device=dev)
        rl = torch.empty(M, N, device=dev)
        with _timed("executor_relu_relax", 0.0, 4.0 * (4 * M * N + 4 * D * N)):
            _lib.call("bf_crown_relu_relax", _lib.ptr(request.A_u), _lib.ptr(request.A_l), S * N, D, S, N,
                      _lib.ptr(table), None, 0, _lib.ptr(kbias), None, None, None, _lib.ptr(ru), _lib.ptr(rl),
                      _lib.ptr(du), _lib.ptr(dl), None, None, st)
        with _timed("executor_conv_transpose", flops, 4.0 * (2 * M * N + 2 * M * Ci * Hi * Wi)):
            _lib.call("bf_conv_transpose_rows", _lib.ptr(ru), _lib.ptr(rl), M, Co, Ho, Wo, _lib.ptr(W), Ci, KH, KW,
                      sh, sw, ph, pw, Hi, Wi, _lib.ptr(pu), _lib.ptr(pl), S, None, 0, 0, None, None, None, None, st)
        return FusedReluAffineResult(pu, pl, du, dl)


def build_fused_crown_runtime_selection(ops: Sequence[Any], *, backend: str,
                                        chunk_rows: int = 512) -> FusedCrownRuntimeSelection:
    """Map a planner backend decision to an executable runtime plan; "hip_fused"
    selects HipFusedCrownExecutor (the reference's TVM/PyTorch backends are not
    part of this package)."""
    del chunk_rows
    if backend in {"pytorch_eager", "pytorch_structured"}:
        return FusedCrownRuntimeSelection(backend=backend, executor=None, steps=())
    if backend != "hip_fused":
        raise ValueError(f"unsupported fused CROWN runtime backend in the HIP package: {backend}")
    return FusedCrownRuntimeSelection(backend=backend, executor=HipFusedCrownExecutor(),
                                      steps=plan_fused_crown_regions(ops, backend=backend))


# The fused Task IR a typed registry hands to this backend: one ReLU relaxation
# followed by one affine backward op (task_backend_dispatch.py:467-472).
_FUSED_TASK_KINDS = ("relu_relaxation", ("linear_backward", "conv2d_backward"))


@dataclass(frozen=True)
class _PreparedHipTask:
    backend: str
    task_id: str
    op_ids: Tuple[str, ...]
    output_value_ids: Tuple[str, ...]
    capability_id: str


class HipTaskBackendRegistry:
    """Typed-registry entry of the ``"hip_fused"`` backend kind.

    Mirrors what ``TVMTaskBackendRegistry.dispatch`` does once the reference's
    ``_validate_typed_dispatch`` has checked the dispatch key against the task
    and plan template (task_backend_dispatch.py:363-402, 435-495): the selected
    backend candidate must be ``"hip_fused"``, the task must be the fused
    ReLU -> Linear / Conv2d pair, a prepared task is cached by the key's stable
    hash (a different task under the same hash is rejected as a collision), and
    the region runs through the session with ``HipFusedCrownExecutor``.  The
    duck-typed arguments are the reference's ``TaskIRUnit``,
    ``BackendDispatchKey``, ``PlainCrownBoundIRSession`` and ``PlanTemplate``."""

    backend = "hip_fused"

    def __init__(self) -> None:
        self._prepared: dict = {}
        self.cache_hits = 0
        self.cache_misses = 0
        self._executor = HipFusedCrownExecutor()

    def dispatch(self, task: Any, key: Any, *, session: Any, template: Any):
        candidates = {c.candidate_id: c for c in template.backend_candidates}
        candidate = candidates.get(key.backend_candidate_id)
        if candidate is None:
            raise ValueError("typed registry dispatch references unknown backend")
        kind = getattr(candidate.backend, "value", candidate.backend)
        if kind != self.backend:
            raise ValueError(f"HIP registry rejects backend: {kind}")
        kinds = tuple(getattr(op.kind, "value", op.kind) for op in task.op_refs)
        if not (len(kinds) == 2 and kinds[0] == _FUSED_TASK_KINDS[0] and kinds[1] in _FUSED_TASK_KINDS[1]):
            raise ValueError("HIP CROWN backend requires fused ReLU->Affine Task IR")
        prepared = _PreparedHipTask(backend=kind, task_id=task.task_id,
                                    op_ids=tuple(op.op_id for op in task.op_refs),
                                    output_value_ids=tuple(task.output_value_ids),
                                    capability_id=candidate.capability_id)
        digest = key.stable_hash()
        cached = self._prepared.get(digest)
        if cached is None:
            self._prepared[digest] = prepared
            self.cache_misses += 1
        elif cached != prepared:
            raise ValueError("HIP backend cache key collision or stale task")
        else:
            self.cache_hits += 1
        return session.execute_fused_relu_affine_task(prepared.op_ids, output_value_ids=prepared.output_value_ids,
                                                      executor=self._executor)
