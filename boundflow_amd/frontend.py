"""PyTorch frontend and planner v0: from an ``nn.Module`` to the task module the
HIP backend runs.

* ``import_torch`` -- boundflow/frontends/pytorch/frontend.py:21-80: the module is
  captured with ``torch.export`` (or ``torch.fx.symbolic_trace``) and every node
  becomes a primal-graph node whose op type is the BoundFlow primitive of its
  ATen target (linear, relu, add, concat, conv2d, matmul, flatten, reshape,
  permute; other targets keep their ATen name), with the constant arguments the
  runtime needs as attrs (conv2d stride/padding/dilation/groups, flatten dims,
  permute dims, concat axis).  Parameters are keyed by their placeholder names.
* ``normalize_primal_graph`` -- boundflow/frontends/normalize.py: tensor-method
  nodes mapped to primitives (view/reshape -> reshape, permute), "transpose" ->
  "permute".
* ``plan_interval_ibp_v0`` -- boundflow/planner/interval_v0.py:10-76: the whole
  graph as one INTERVAL_IBP task, affine ops tagged with ``attrs["op"]``,
  reshape targets taken from the value shapes, layout-only permutes composed or
  dropped (boundflow/planner/passes/layout_only.py), and one buffer per value.

The primal IR dataclasses carry the reference's fields
(boundflow/ir/primal.py): they are the frontend's output contract.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from typing import Any, Dict, Iterable, List, Optional, Tuple

import torch

from .ir import BFTaskModule, BoundTask, BufferSpec, StoragePlan, TaskKind, TaskLowering, TaskOp


# ---------------------------------------------------------------------------
# Primal IR (boundflow/ir/primal.py)


class Source(Enum):
    TORCH_EXPORT = "torch_export"
    ONNX = "onnx"


class ValueKind(Enum):
    INPUT = "input"
    PARAM = "param"
    CONST = "const"
    INTERMEDIATE = "intermediate"


@dataclass(frozen=True)
class TensorType:
    shape: List[Optional[int]]
    dtype: str
    layout: Optional[str] = None


@dataclass
class Value:
    """A data edge of the graph (an SSA value) with its shape and dtype."""

    name: str
    type: TensorType
    kind: ValueKind = ValueKind.INTERMEDIATE
    debug_name: Optional[str] = None


@dataclass
class Node:
    """An operation; inputs and outputs are value names."""

    op_type: str
    name: str
    inputs: List[str]
    outputs: List[str]
    attrs: Dict[str, Any] = field(default_factory=dict)


@dataclass
class BFPrimalGraph:
    nodes: List[Node] = field(default_factory=list)
    inputs: List[str] = field(default_factory=list)
    outputs: List[str] = field(default_factory=list)
    values: Dict[str, Value] = field(default_factory=dict)

    def validate(self) -> None:
        names = [n.name for n in self.nodes]
        if len(set(names)) != len(names):
            dup = next(n for n in names if names.count(n) > 1)
            raise ValueError(f"duplicate node name: {dup}")
        for v in self.inputs + self.outputs:
            if v not in self.values:
                raise ValueError(f"graph input/output value missing meta: {v}")
        for node in self.nodes:
            for v in node.inputs + node.outputs:
                if v not in self.values:
                    raise ValueError(f"node '{node.name}' references unknown value: {v}")


@dataclass
class BFPrimalProgram:
    source: Source
    graph: BFPrimalGraph
    params: Dict[str, Any]
    tensor_meta: Dict[str, Any]
    debug_map: Dict[str, str] = field(default_factory=dict)


# ---------------------------------------------------------------------------
# torch -> primal graph

# ATen overload -> BoundFlow primitive
_PRIMITIVES = {
    "aten.linear.default": "linear",
    "aten.relu.default": "relu",
    "aten.add.Tensor": "add",
    "aten.cat.default": "concat",
    "aten.concat.default": "concat",
    "aten.conv2d.default": "conv2d",
    "aten.matmul.default": "matmul",
    "aten.flatten.using_ints": "flatten",
    "aten.reshape.default": "reshape",
    "aten.view.default": "reshape",
    "aten.permute.default": "permute",
}

_METHODS = {"view": "reshape", "reshape": "reshape", "permute": "permute"}


def _target_name(target: Any) -> str:
    try:
        return str(target)
    except Exception:   # a target without a printable form
        return getattr(target, "__name__", "<unknown>")


def _tensor_type(node: "torch.fx.Node", fallback: Any = None) -> TensorType:
    meta = node.meta.get("tensor_meta")
    src = meta if meta is not None else fallback
    if src is not None and hasattr(src, "shape") and hasattr(src, "dtype"):
        return TensorType(shape=[None if d is None else int(d) for d in src.shape],
                          dtype=str(src.dtype).replace("torch.", ""))
    return TensorType(shape=[], dtype="unknown")


def _node_refs(obj: Any) -> List[str]:
    """Names of the fx nodes an argument structure refers to, in order."""
    if isinstance(obj, torch.fx.Node):
        return [obj.name]
    if isinstance(obj, (list, tuple)):
        return [name for item in obj for name in _node_refs(item)]
    if isinstance(obj, dict):
        return [name for item in obj.values() for name in _node_refs(item)]
    return []


def _call_attrs(op: str, node: "torch.fx.Node") -> Dict[str, Any]:
    """Constant arguments of a call the runtime reads as attrs."""
    args = list(node.args)

    def arg(i, default):
        return args[i] if len(args) > i else default

    if op == "conv2d":
        # aten.conv2d(input, weight, bias, stride, padding, dilation, groups)
        return {"stride": arg(3, 1), "padding": arg(4, 0), "dilation": arg(5, 1), "groups": arg(6, 1)}
    if op == "flatten":
        return {"start_dim": int(arg(1, 0)), "end_dim": int(arg(2, -1))}
    if op in ("permute", "transpose"):
        dims = arg(1, None)
        if not isinstance(dims, (list, tuple)):
            raise ValueError(f"permute dims must be list/tuple, got {type(dims)}: {dims}")
        return {"dims": [int(d) for d in dims]}
    if op == "concat":
        axis = node.kwargs.get("dim", arg(1, 0))
        return {"axis": int(axis if axis is not None else 0)}
    return {}


def _attr_value(gm: "torch.fx.GraphModule", target: Any) -> Any:
    obj: Any = gm
    for part in str(target).split("."):
        obj = getattr(obj, part)
    return obj


def _graph_from_fx(gm: "torch.fx.GraphModule", *, user_inputs: List[str], param_placeholders: Dict[str, str],
                   consts: Dict[str, Any]) -> BFPrimalGraph:
    g = BFPrimalGraph()
    for node in gm.graph.nodes:
        if node.op == "placeholder":
            kind = (ValueKind.PARAM if node.name in param_placeholders else
                    ValueKind.INPUT if node.name in user_inputs else ValueKind.INTERMEDIATE)
            g.values[node.name] = Value(node.name, _tensor_type(node), kind, str(node.target))
        elif node.op == "get_attr":
            val = _attr_value(gm, node.target)
            consts[node.name] = val
            g.values[node.name] = Value(node.name, _tensor_type(node, val), ValueKind.CONST, str(node.target))
        elif node.op in ("call_function", "call_method"):
            if node.op == "call_function":
                op = _PRIMITIVES.get(_target_name(node.target), _target_name(node.target))
                attrs = _call_attrs(op, node)
            else:
                op = f"call_method::{node.target}"
                attrs = {}
            g.nodes.append(Node(op, node.name, _node_refs(node.args) + _node_refs(node.kwargs), [node.name], attrs))
            g.values[node.name] = Value(node.name, _tensor_type(node), ValueKind.INTERMEDIATE,
                                        _target_name(node.target))
        elif node.op == "output":
            g.outputs = _node_refs(node.args)
        else:
            raise NotImplementedError(f"unsupported fx node op: {node.op}")
    g.inputs = list(user_inputs)
    g.validate()
    return g


def normalize_primal_graph(graph: BFPrimalGraph) -> BFPrimalGraph:
    """Tensor-method nodes to primitives; "transpose" to "permute" (in place)."""
    graph.validate()
    for node in graph.nodes:
        if node.op_type.startswith("call_method::"):
            method = node.op_type.split("::", 1)[1]
            node.op_type = _METHODS.get(method, node.op_type)
        if node.op_type == "transpose":
            node.op_type = "permute"
    return graph


def import_torch(module: torch.nn.Module, example_inputs: Tuple[Any, ...], *, strict: bool = False,
                 normalize: bool = True, export_mode: str = "export") -> BFPrimalProgram:
    """Capture ``module`` on ``example_inputs`` as a primal program (frontend.py:21-80).
    ``export_mode`` "export" uses torch.export (parameters become PARAM placeholders
    and ``params``), "fx" symbolic tracing (parameters stay get_attr constants)."""
    if export_mode not in ("export", "fx"):
        raise ValueError(f"unsupported export_mode: {export_mode}")
    consts: Dict[str, Any] = {}
    if export_mode == "fx":
        gm = torch.fx.symbolic_trace(module)
        # the user inputs are the placeholders in order, under their own names (the reference
        # names them arg0, arg1, ..., which matches only forward(self, arg0, ...) signatures)
        placeholders = [n.name for n in gm.graph.nodes if n.op == "placeholder"][:len(example_inputs)]
        graph = _graph_from_fx(gm, user_inputs=placeholders, param_placeholders={}, consts=consts)
        program = BFPrimalProgram(Source.TORCH_EXPORT, graph, {}, {"export_mode": "fx"})
    else:
        ep = torch.export.export(module, tuple(example_inputs), strict=strict)
        sig = ep.graph_signature
        to_param = dict(sig.inputs_to_parameters)
        state = dict(ep.state_dict)
        graph = _graph_from_fx(ep.graph_module, user_inputs=list(sig.user_inputs), param_placeholders=to_param,
                               consts=consts)
        params = {ph: state[tgt] for ph, tgt in to_param.items() if tgt in state}
        meta = {"inputs_to_parameters": to_param, "inputs_to_buffers": dict(getattr(sig, "inputs_to_buffers", {})),
                "user_inputs": list(sig.user_inputs), "user_outputs": list(sig.user_outputs)}
        program = BFPrimalProgram(Source.TORCH_EXPORT, graph, params,
                                  {"export_mode": "export", "graph_signature": meta})
    if normalize:
        program.graph = normalize_primal_graph(program.graph)
    return program


# ---------------------------------------------------------------------------
# planner v0


def simplify_layout_only_ops(ops: List[TaskOp], *, output_values: List[str]) -> Tuple[List[TaskOp], List[str]]:
    """Drop identity permutes and compose consecutive ones
    (boundflow/planner/passes/layout_only.py); consumers of a removed value read
    its source through an alias map."""
    alias: Dict[str, str] = {}

    def resolve(v: str) -> str:
        while v in alias:
            v = alias[v]
        return v

    def dims_of(attrs) -> Optional[List[int]]:
        dims = attrs.get("dims")
        if not isinstance(dims, (list, tuple)):
            return None
        try:
            return [int(d) for d in dims]
        except (TypeError, ValueError):
            return None

    out: List[TaskOp] = []
    for op in ops:
        ins = [resolve(v) for v in op.inputs]
        kind = "permute" if op.op_type == "transpose" else op.op_type
        dims = dims_of(op.attrs) if kind == "permute" else None
        if kind != "permute" or len(ins) != 1 or len(op.outputs) != 1 or dims is None:
            out.append(TaskOp(op_type=kind, name=op.name, inputs=ins, outputs=list(op.outputs), attrs=dict(op.attrs)))
            continue
        src, dst = ins[0], op.outputs[0]
        if dims == list(range(len(dims))):
            alias[dst] = src
            continue
        prev = out[-1] if out else None
        if (prev is not None and prev.op_type == "permute" and len(prev.outputs) == 1 and prev.outputs[0] == src
                and len(prev.inputs) == 1 and dims_of(prev.attrs) is not None):
            composed = [dims_of(prev.attrs)[d] for d in dims]
            if composed == list(range(len(composed))):
                out.pop()
                alias[prev.outputs[0]] = prev.inputs[0]
                alias[dst] = prev.inputs[0]
            else:
                prev.attrs = dict(prev.attrs)
                prev.attrs["dims"] = composed
                prev.attrs.setdefault("layout_only", True)
                alias[dst] = prev.outputs[0]
            continue
        attrs = dict(op.attrs)
        attrs["dims"] = dims
        attrs.setdefault("layout_only", True)
        out.append(TaskOp(op_type="permute", name=op.name, inputs=[src], outputs=[dst], attrs=attrs))
    outputs: List[str] = []
    for v in (resolve(v) for v in output_values):
        if v not in outputs:
            outputs.append(v)
    return out, outputs


def _buffer_scope(value: Value) -> str:
    return {ValueKind.PARAM: "param", ValueKind.CONST: "const"}.get(value.kind, "global")


def _unique(xs: Iterable[str]) -> List[str]:
    out: List[str] = []
    for x in xs:
        if x not in out:
            out.append(x)
    return out


def plan_interval_ibp_v0(program: BFPrimalProgram) -> BFTaskModule:
    """The whole primal graph as one interval-IBP task (interval_v0.py:10-76)."""
    graph = program.graph
    graph.validate()
    ops = []
    for node in graph.nodes:
        attrs = dict(node.attrs)
        if node.op_type in ("linear", "conv2d"):
            attrs.setdefault("op", node.op_type)
        if node.op_type == "reshape":
            val = graph.values.get(node.outputs[0])
            if val is not None and val.type.shape:
                attrs.setdefault("shape", [-1 if d is None else int(d) for d in val.type.shape])
        ops.append(TaskOp(op_type=node.op_type, name=node.name, inputs=list(node.inputs),
                          outputs=list(node.outputs), attrs=attrs))
    ops, outputs = simplify_layout_only_ops(ops, output_values=list(graph.outputs))
    plan = StoragePlan()
    for name, val in graph.values.items():
        bid = f"buf_{name}"
        plan.buffers[bid] = BufferSpec(buffer_id=bid, dtype=val.type.dtype, shape=list(val.type.shape),
                                       scope=_buffer_scope(val), device=None, layout=val.type.layout)
        plan.value_to_buffer[name] = bid
    task = BoundTask(
        task_id="ibp_task0",
        kind=TaskKind.INTERVAL_IBP,
        ops=ops,
        input_values=list(graph.inputs),
        output_values=outputs,
        input_buffers=_unique(plan.value_to_buffer[v] for v in graph.inputs if v in plan.value_to_buffer),
        output_buffers=_unique(plan.value_to_buffer[v] for v in outputs if v in plan.value_to_buffer),
        params=list(program.params.keys()),
        batch_axes={},
        memory_plan={},
        lowering=TaskLowering.TVM_TIR,
    )
    module = BFTaskModule(tasks=[task], entry_task_id=task.task_id,
                          bindings={"params": dict(program.params), "tensor_meta": dict(program.tensor_meta)},
                          storage_plan=plan)
    module.validate()
    return module
