"""Task IR consumed by the HIP backend.

These dataclasses carry the same fields and validation rules as the reference
planner's output so that a BoundTask list and its StoragePlan can be handed to
this backend unchanged:

* ``TaskKind``/``TaskLowering``/``MemoryEffect`` -- boundflow/ir/task.py:14-28
* ``BufferSpec`` -- boundflow/ir/task.py:31-49
* ``StoragePlan`` (logical/physical buffer map) -- boundflow/ir/task.py:52-116
* ``TaskOp`` -- boundflow/ir/task.py:119-132
* ``BoundTask`` -- boundflow/ir/task.py:135-173
* ``BFTaskModule`` -- boundflow/ir/task.py:176-240
* ``TaskBufferDep``/``TaskDepEdge``/``TaskGraph`` -- boundflow/ir/task_graph.py:11-168

Only the planner-visible contract lives here; nothing in this module touches
the device.
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass, field
from enum import Enum
from typing import Any, Dict, List, Optional, Set


class TaskKind(Enum):
    INTERVAL_IBP = "interval_ibp"


class TaskLowering(Enum):
    TVM_TIR = "tvm_tir"
    CONSTRAINT = "constraint"
    HIP = "hip"


class MemoryEffect(Enum):
    READ = "read"
    WRITE = "write"
    READWRITE = "readwrite"
    ALLOC = "alloc"
    FREE = "free"


@dataclass(frozen=True)
class BufferSpec:
    """One logical or physical buffer (boundflow/ir/task.py:31-49)."""

    buffer_id: str
    dtype: str
    shape: List[Optional[int]]
    scope: str = "global"
    device: Optional[str] = None
    layout: Optional[str] = None
    strides: Optional[List[int]] = None
    alignment: Optional[int] = None
    alias_group: Optional[str] = None


@dataclass
class StoragePlan:
    """value -> logical buffer -> physical buffer map (boundflow/ir/task.py:52-116)."""

    buffers: Dict[str, BufferSpec] = field(default_factory=dict)
    value_to_buffer: Dict[str, str] = field(default_factory=dict)
    physical_buffers: Dict[str, BufferSpec] = field(default_factory=dict)
    logical_to_physical: Dict[str, str] = field(default_factory=dict)

    def to_physical(self, logical_buffer_id: str) -> str:
        return self.logical_to_physical.get(logical_buffer_id, logical_buffer_id)

    def get_logical_spec(self, logical_buffer_id: str) -> BufferSpec:
        if logical_buffer_id not in self.buffers:
            raise KeyError(f"logical buffer_id not found: {logical_buffer_id}")
        return self.buffers[logical_buffer_id]

    def get_physical_spec(self, logical_buffer_id: str) -> BufferSpec:
        phys = self.to_physical(logical_buffer_id)
        if self.physical_buffers:
            if phys not in self.physical_buffers:
                raise KeyError(f"physical buffer_id not found: {phys} (from logical {logical_buffer_id})")
            return self.physical_buffers[phys]
        return self.get_logical_spec(phys)

    def num_logical_buffers(self) -> int:
        return len(self.buffers)

    def num_physical_buffers(self) -> int:
        return len(self.physical_buffers) if self.physical_buffers else len(self.buffers)

    def validate(self) -> None:
        for value_name, buffer_id in self.value_to_buffer.items():
            if buffer_id not in self.buffers:
                raise ValueError(f"storage_plan references missing buffer_id: {buffer_id} (value={value_name})")
        for logical_id, physical_id in self.logical_to_physical.items():
            if logical_id not in self.buffers:
                raise ValueError(f"logical_to_physical references missing logical buffer_id: {logical_id}")
            if self.physical_buffers:
                if physical_id not in self.physical_buffers:
                    raise ValueError(
                        f"logical_to_physical references missing physical buffer_id: {physical_id} (logical={logical_id})"
                    )
            elif physical_id != logical_id:
                raise ValueError(
                    "logical_to_physical is non-identity but physical_buffers is empty; "
                    f"logical={logical_id} physical={physical_id}"
                )
        for bid, spec in self.physical_buffers.items():
            if spec.buffer_id != bid:
                raise ValueError(f"physical_buffers spec.buffer_id mismatch: key={bid} spec={spec.buffer_id}")


@dataclass
class TaskOp:
    """One primitive of a task; inputs/outputs are value names (boundflow/ir/task.py:119-132)."""

    op_type: str
    name: str
    inputs: List[str]
    outputs: List[str]
    attrs: Dict[str, Any] = field(default_factory=dict)
    memory_effect: Optional[MemoryEffect] = None


@dataclass
class BoundTask:
    """A planner task (boundflow/ir/task.py:135-173)."""

    task_id: str
    kind: TaskKind
    ops: List[TaskOp]
    input_values: List[str]
    output_values: List[str]
    input_buffers: List[str] = field(default_factory=list)
    output_buffers: List[str] = field(default_factory=list)
    batch_axes: Dict[str, str] = field(default_factory=dict)
    memory_plan: Dict[str, Any] = field(default_factory=dict)
    lowering: TaskLowering = TaskLowering.TVM_TIR
    target_func_name: str = ""
    params: List[str] = field(default_factory=list)

    def validate(self) -> None:
        if not self.task_id:
            raise ValueError("task_id must be non-empty")
        if not self.ops:
            raise ValueError(f"task '{self.task_id}' has no ops")
        if not self.input_values:
            raise ValueError(f"task '{self.task_id}' has no inputs")
        if not self.output_values:
            raise ValueError(f"task '{self.task_id}' has no outputs")
        if len(set(self.input_buffers)) != len(self.input_buffers):
            raise ValueError(f"task '{self.task_id}' has duplicate input_buffers")
        if len(set(self.output_buffers)) != len(self.output_buffers):
            raise ValueError(f"task '{self.task_id}' has duplicate output_buffers")


@dataclass
class BFTaskModule:
    """Container for the executable task list (boundflow/ir/task.py:176-240)."""

    tasks: List[BoundTask]
    entry_task_id: str
    tvm_mod: Optional[Any] = None
    bindings: Dict[str, Any] = field(default_factory=dict)
    storage_plan: StoragePlan = field(default_factory=StoragePlan)
    task_graph: Optional[Any] = None

    def get_task(self, task_id: str) -> BoundTask:
        for task in self.tasks:
            if task.task_id == task_id:
                return task
        raise KeyError(f"task_id not found: {task_id}")

    def get_entry_task(self) -> BoundTask:
        return self.get_task(self.entry_task_id)

    def validate(self) -> None:
        if not self.tasks:
            raise ValueError("BFTaskModule.tasks must be non-empty")
        ids = [t.task_id for t in self.tasks]
        if len(set(ids)) != len(ids):
            raise ValueError("duplicate task_id in BFTaskModule")
        self.get_entry_task()
        for task in self.tasks:
            task.validate()
        self.storage_plan.validate()
        if self.task_graph is not None:
            for task in self.tasks:
                if not task.input_buffers:
                    raise ValueError(f"task '{task.task_id}' missing input_buffers (required when task_graph exists)")
                if not task.output_buffers:
                    raise ValueError(f"task '{task.task_id}' missing output_buffers (required when task_graph exists)")
                for v in task.input_values:
                    b = self.storage_plan.value_to_buffer.get(v)
                    if b is None or b not in task.input_buffers:
                        raise ValueError(f"task '{task.task_id}' input_buffers missing buffer for value '{v}'")
                for v in task.output_values:
                    b = self.storage_plan.value_to_buffer.get(v)
                    if b is None or b not in task.output_buffers:
                        raise ValueError(f"task '{task.task_id}' output_buffers missing buffer for value '{v}'")
            self.task_graph.validate(tasks_by_id={t.task_id: t for t in self.tasks},
                                     entry_task_id=self.entry_task_id, storage_plan=self.storage_plan)

    @property
    def params(self) -> Dict[str, Any]:
        raw = self.bindings.get("params", {})
        return dict(raw) if isinstance(raw, dict) else {}


@dataclass(frozen=True)
class TaskBufferDep:
    """One value handed from a producer task to a consumer task, with the
    buffers both sides bind it to (task_graph.py:11-20)."""

    src_value: str
    src_buffer_id: str
    dst_value: str
    dst_buffer_id: str


@dataclass(frozen=True)
class TaskDepEdge:
    """Producer -> consumer task edge at buffer granularity (task_graph.py:23-34)."""

    src_task_id: str
    dst_task_id: str
    deps: List[TaskBufferDep]


@dataclass
class TaskGraph:
    """DAG of BoundTasks scheduled in topological order (task_graph.py:37-168)."""

    task_ids: List[str]
    edges: List[TaskDepEdge] = field(default_factory=list)

    def validate(self, *, tasks_by_id: Dict[str, BoundTask], entry_task_id: str, storage_plan: StoragePlan) -> None:
        if entry_task_id not in tasks_by_id:
            raise KeyError(f"entry_task_id not found in tasks: {entry_task_id}")
        if not self.task_ids:
            raise ValueError("TaskGraph.task_ids must be non-empty")
        if len(set(self.task_ids)) != len(self.task_ids):
            raise ValueError("TaskGraph.task_ids contains duplicates")
        missing = [t for t in self.task_ids if t not in tasks_by_id]
        if missing:
            raise KeyError(f"TaskGraph references missing task_id: {missing[0]}")
        for edge in self.edges:
            for end in (edge.src_task_id, edge.dst_task_id):
                if end not in tasks_by_id:
                    raise KeyError(f"edge task_id missing: {end}")
            src, dst = tasks_by_id[edge.src_task_id], tasks_by_id[edge.dst_task_id]
            for dep in edge.deps:
                if dep.src_value not in src.output_values:
                    raise ValueError(f"edge src_value '{dep.src_value}' not in src task outputs: {src.task_id}")
                if dep.dst_value not in dst.input_values:
                    raise ValueError(f"edge dst_value '{dep.dst_value}' not in dst task inputs: {dst.task_id}")
                for value, bid, task, side in ((dep.src_value, dep.src_buffer_id, src, "output"),
                                               (dep.dst_value, dep.dst_buffer_id, dst, "input")):
                    if bid not in storage_plan.buffers:
                        raise ValueError(f"edge buffer missing in storage_plan: {bid}")
                    bound = task.output_buffers if side == "output" else task.input_buffers
                    if bound and bid not in bound:
                        raise ValueError(f"edge buffer '{bid}' not in task {side}_buffers: {task.task_id}")
                    if storage_plan.value_to_buffer.get(value) != bid:
                        raise ValueError(f"edge value->buffer mismatch: {value} -> "
                                         f"{storage_plan.value_to_buffer.get(value)} (edge expects {bid})")
        self.topo_sort(tasks_by_id=tasks_by_id, entry_task_id=entry_task_id)

    def reachable_from(self, entry_task_id: str) -> Set[str]:
        succ: Dict[str, List[str]] = {}
        for e in self.edges:
            succ.setdefault(e.src_task_id, []).append(e.dst_task_id)
        seen: Set[str] = set()
        todo = [entry_task_id]
        while todo:
            t = todo.pop()
            if t not in seen:
                seen.add(t)
                todo.extend(n for n in succ.get(t, []) if n not in seen)
        return seen

    def topo_sort(self, *, tasks_by_id: Dict[str, BoundTask], entry_task_id: str) -> List[str]:
        """Kahn's algorithm over the subgraph reachable from the entry task; ready
        tasks leave in lexicographic order, so the order is deterministic."""
        reachable = self.reachable_from(entry_task_id)
        indeg = {t: 0 for t in reachable}
        succ: Dict[str, List[str]] = {t: [] for t in reachable}
        for e in self.edges:
            if e.src_task_id in reachable and e.dst_task_id in reachable:
                succ[e.src_task_id].append(e.dst_task_id)
                indeg[e.dst_task_id] += 1
        ready = sorted(t for t, d in indeg.items() if d == 0)
        heapq.heapify(ready)
        order: List[str] = []
        while ready:
            t = heapq.heappop(ready)
            order.append(t)
            for n in succ[t]:
                indeg[n] -= 1
                if indeg[n] == 0:
                    heapq.heappush(ready, n)
        if len(order) != len(reachable):
            raise ValueError(f"TaskGraph contains a cycle in reachable subgraph: {sorted(reachable)}")
        for t in order:
            if t not in tasks_by_id:
                raise KeyError(f"topo_sort referenced missing task_id: {t}")
        return order

    @staticmethod
    def chain(*task_ids: str, deps: Optional[List[TaskBufferDep]] = None) -> "TaskGraph":
        """t0 -> t1 -> ... -> tn, every edge carrying ``deps``."""
        if not task_ids:
            raise ValueError("TaskGraph.chain expects at least one task_id")
        edges = [TaskDepEdge(src_task_id=a, dst_task_id=b, deps=list(deps or []))
                 for a, b in zip(task_ids[:-1], task_ids[1:])]
        return TaskGraph(task_ids=list(task_ids), edges=edges)


def default_storage_plan(values: List[str], *, dtype: str = "float32") -> StoragePlan:
    """One buffer per value, the layout ``plan_interval_ibp_v0`` emits
    (boundflow/planner/interval_v0.py:78-106)."""

    plan = StoragePlan()
    for v in values:
        bid = f"buf_{v}"
        plan.buffers[bid] = BufferSpec(buffer_id=bid, dtype=dtype, shape=[None])
        plan.value_to_buffer[v] = bid
    return plan
