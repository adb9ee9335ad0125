"""Seeded synthetic workloads for the five benchmark configurations.

Everything is generated on the CPU from one ``torch.Generator`` so that the
HIP path and the CPU baseline see bit-identical inputs.  Networks are built
directly as ``BFTaskModule`` programs with the op vocabulary the reference's
planner emits (``linear``/``conv2d``/``relu``/``flatten``), one task, one
buffer per value.

Configurations (shapes, distributions and optimiser settings):

* C1  IBP+CROWN, MLP 784-256-256-10, B=64, box eps=2/255 clamped to [0,1]
* C2  CROWN with all intermediate bounds by CROWN, MLP 784-500x6-10, B=256, Linf 0.015
* C3  CROWN, CNN 3x32x32 conv(16,4,s2,p1)-conv(32,4,s2,p1)-fc100-fc10, B=128, Linf 2/255
* C4  alpha-CROWN on the C3 CNN, B=32, Linf 8/255, 20 Adam steps, lr 0.1, alpha from CROWN
* C5  beta-CROWN BaB domain batch, MLP 784-256x4-10, 4096 domains from one input,
      Linf 0.03, 1-12 random unstable-neuron splits per domain, 10 steps

Weights are Kaiming (uniform for C1/C3/C4/C5, normal for C2, relu gain);
biases are 0 except C2 (N(0, 0.01^2)).  Specs are the 9 margin rows
``e_y - e_j`` of a random true label ``y``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from .ir import (BFTaskModule, BoundTask, BufferSpec, StoragePlan, TaskBufferDep, TaskDepEdge, TaskGraph, TaskKind,
                 TaskOp, default_storage_plan)
from .spec import InputSpec


@dataclass
class Workload:
    name: str
    module: BFTaskModule
    spec: InputSpec
    C: torch.Tensor
    labels: torch.Tensor
    extra: Dict[str, object] = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return int(self.spec.center.shape[0])

    @property
    def num_specs(self) -> int:
        return int(self.C.shape[1])


def _kaiming(shape, *, fan_in: int, gen: torch.Generator, kind: str) -> torch.Tensor:
    gain = math.sqrt(2.0)
    std = gain / math.sqrt(fan_in)
    if kind == "uniform":
        bound = math.sqrt(3.0) * std
        return (torch.rand(shape, generator=gen, dtype=torch.float64) * 2.0 - 1.0).mul_(bound).to(torch.float32)
    return (torch.randn(shape, generator=gen, dtype=torch.float64) * std).to(torch.float32)


def build_mlp(dims: Sequence[int], *, gen: torch.Generator, init: str = "uniform",
              bias_std: float = 0.0) -> BFTaskModule:
    """Chain MLP ``dims[0] -> ... -> dims[-1]`` with ReLU between linear layers."""
    ops: List[TaskOp] = []
    params: Dict[str, torch.Tensor] = {}
    prev = "input"
    values = ["input"]
    n = len(dims) - 1
    for i in range(n):
        W = _kaiming((dims[i + 1], dims[i]), fan_in=dims[i], gen=gen, kind=init)
        if bias_std > 0:
            b = (torch.randn(dims[i + 1], generator=gen, dtype=torch.float64) * bias_std).to(torch.float32)
        else:
            b = torch.zeros(dims[i + 1], dtype=torch.float32)
        params[f"W{i}"] = W
        params[f"b{i}"] = b
        out = "out" if i == n - 1 else f"h{i}"
        ops.append(TaskOp(op_type="linear", name=f"linear{i}", inputs=[prev, f"W{i}", f"b{i}"], outputs=[out]))
        values.append(out)
        if i < n - 1:
            r = f"r{i}"
            ops.append(TaskOp(op_type="relu", name=f"relu{i}", inputs=[out], outputs=[r]))
            values.append(r)
            prev = r
    return _module(ops, params, values)


def build_cnn(*, gen: torch.Generator) -> BFTaskModule:
    """3x32x32 -> conv(16,4,s2,p1) -> relu -> conv(32,4,s2,p1) -> relu -> flatten -> fc100 -> relu -> fc10."""
    ops: List[TaskOp] = []
    params: Dict[str, torch.Tensor] = {}
    params["W0"] = _kaiming((16, 3, 4, 4), fan_in=3 * 16, gen=gen, kind="uniform")
    params["b0"] = torch.zeros(16)
    params["W1"] = _kaiming((32, 16, 4, 4), fan_in=16 * 16, gen=gen, kind="uniform")
    params["b1"] = torch.zeros(32)
    params["W2"] = _kaiming((100, 2048), fan_in=2048, gen=gen, kind="uniform")
    params["b2"] = torch.zeros(100)
    params["W3"] = _kaiming((10, 100), fan_in=100, gen=gen, kind="uniform")
    params["b3"] = torch.zeros(10)
    conv = {"stride": 2, "padding": 1, "dilation": 1, "groups": 1}
    ops.append(TaskOp("conv2d", "conv0", ["input", "W0", "b0"], ["h0"], dict(conv)))
    ops.append(TaskOp("relu", "relu0", ["h0"], ["r0"]))
    ops.append(TaskOp("conv2d", "conv1", ["r0", "W1", "b1"], ["h1"], dict(conv)))
    ops.append(TaskOp("relu", "relu1", ["h1"], ["r1"]))
    ops.append(TaskOp("flatten", "flatten", ["r1"], ["f1"], {"start_dim": 1, "end_dim": -1}))
    ops.append(TaskOp("linear", "linear2", ["f1", "W2", "b2"], ["h2"]))
    ops.append(TaskOp("relu", "relu2", ["h2"], ["r2"]))
    ops.append(TaskOp("linear", "linear3", ["r2", "W3", "b3"], ["out"]))
    values = ["input", "h0", "r0", "h1", "r1", "f1", "h2", "r2", "out"]
    return _module(ops, params, values)


def _bias(n: int, gen: torch.Generator, std: float) -> torch.Tensor:
    return (torch.randn(n, generator=gen, dtype=torch.float64) * std).to(torch.float32)


DAG_KINDS = ("residual_mlp", "projection_skip_cnn", "feature_concat_mlp", "channel_concat_cnn")


def build_dag(kind: str, *, gen: torch.Generator, n_in: int = 16, hidden: int = 24, n_out: int = 10,
              channels: Tuple[int, int, int] = (2, 6, 6), blocks: int = 1, bias_std: float = 0.1,
              width: Optional[int] = None) -> BFTaskModule:
    """The four DAG shapes of the reference's general-DAG tests
    (tests/test_phase7a_pr8_general_dag_runtime.py:17-237), with Kaiming weights
    and small random biases:

    * ``residual_mlp``: input -> linear -> relu -> linear -> add(input, .) -> relu,
      ``blocks`` times (each block adds its own input), then a linear head; with
      ``width`` a linear + relu stem maps the input to ``width`` features first;
    * ``projection_skip_cnn``: conv(input) -> relu, plus a skip conv of the input,
      add -> relu -> flatten -> linear (C x 8 x 8 input, 3x3 convs, padding 1);
    * ``feature_concat_mlp``: two linear -> relu branches of the input, concat -> linear;
    * ``channel_concat_cnn``: two conv -> relu branches of the input, channel concat
      -> flatten -> linear.
    """
    ops: List[TaskOp] = []
    params: Dict[str, torch.Tensor] = {}
    values = ["input"]

    def lin(name, x, n_from, n_to, out):
        params[f"W_{name}"] = _kaiming((n_to, n_from), fan_in=n_from, gen=gen, kind="uniform")
        params[f"b_{name}"] = _bias(n_to, gen, bias_std)
        ops.append(TaskOp("linear", name, [x, f"W_{name}", f"b_{name}"], [out]))
        values.append(out)

    def conv(name, x, c_from, c_to, out):
        params[f"W_{name}"] = _kaiming((c_to, c_from, 3, 3), fan_in=c_from * 9, gen=gen, kind="uniform")
        params[f"b_{name}"] = _bias(c_to, gen, bias_std)
        ops.append(TaskOp("conv2d", name, [x, f"W_{name}", f"b_{name}"], [out],
                          {"stride": 1, "padding": 1, "dilation": 1, "groups": 1}))
        values.append(out)

    def op(t, name, ins, out, attrs=None):
        ops.append(TaskOp(t, name, ins, [out], dict(attrs or {})))
        values.append(out)

    if kind == "residual_mlp":
        x = "input"
        n = n_in
        if width is not None:
            lin("stem", x, n_in, width, "h_stem")
            op("relu", "relu_stem", ["h_stem"], "r_stem")
            x, n = "r_stem", width
        for i in range(blocks):
            lin(f"lin{i}a", x, n, hidden, f"h{i}a")
            op("relu", f"relu{i}a", [f"h{i}a"], f"r{i}a")
            lin(f"lin{i}b", f"r{i}a", hidden, n, f"h{i}b")
            op("add", f"add{i}", [x, f"h{i}b"], f"s{i}")
            op("relu", f"relu{i}", [f"s{i}"], f"r{i}")
            x = f"r{i}"
        lin("head", x, n, n_out, "out")
    elif kind == "projection_skip_cnn":
        c_in, c_mid, _ = channels
        conv("conv_main", "input", c_in, c_mid, "h_main")
        op("relu", "relu_main", ["h_main"], "r_main")
        conv("conv_skip", "input", c_in, c_mid, "h_skip")
        op("add", "add0", ["r_main", "h_skip"], "sum0")
        op("relu", "relu_out", ["sum0"], "r_out")
        op("flatten", "flatten0", ["r_out"], "flat", {"start_dim": 1, "end_dim": -1})
        lin("head", "flat", c_mid * 64, n_out, "out")
    elif kind == "feature_concat_mlp":
        lin("lin1", "input", n_in, hidden, "h1")
        op("relu", "relu1", ["h1"], "r1")
        lin("lin2", "input", n_in, hidden // 2, "h2")
        op("relu", "relu2", ["h2"], "r2")
        op("concat", "concat0", ["r1", "r2"], "cat0", {"axis": 1})
        lin("head", "cat0", hidden + hidden // 2, n_out, "out")
    elif kind == "channel_concat_cnn":
        c_in, c1, c2 = channels
        conv("conv1", "input", c_in, c1, "h1")
        op("relu", "relu1", ["h1"], "r1")
        conv("conv2", "input", c_in, c2, "h2")
        op("relu", "relu2", ["h2"], "r2")
        op("concat", "concat0", ["r1", "r2"], "cat0", {"axis": 1})
        op("flatten", "flatten0", ["cat0"], "flat", {"start_dim": 1, "end_dim": -1})
        lin("head", "flat", (c1 + c2) * 64, n_out, "out")
    else:
        raise ValueError(f"unknown DAG kind {kind!r}; expected one of {DAG_KINDS}")
    return _module(ops, params, values)


def dag_input_shape(kind: str, *, n_in: int = 16, channels: Tuple[int, int, int] = (2, 6, 6)) -> Tuple[int, ...]:
    return (channels[0], 8, 8) if kind.endswith("_cnn") else (n_in,)


def _module(ops: List[TaskOp], params: Dict[str, torch.Tensor], values: List[str]) -> BFTaskModule:
    task = BoundTask(task_id="t0", kind=TaskKind.INTERVAL_IBP, ops=ops, input_values=["input"],
                     output_values=["out"], params=list(params.keys()))
    return BFTaskModule(tasks=[task], entry_task_id="t0", bindings={"params": params},
                        storage_plan=default_storage_plan(values))


def margin_spec(labels: torch.Tensor, num_classes: int = 10) -> torch.Tensor:
    """C[b] rows are e_y - e_j for every j != y, ordered by j."""
    B = int(labels.shape[0])
    C = torch.zeros(B, num_classes - 1, num_classes)
    for b in range(B):
        y = int(labels[b])
        r = 0
        for j in range(num_classes):
            if j == y:
                continue
            C[b, r, y] = 1.0
            C[b, r, j] = -1.0
            r += 1
    return C


def predicted_labels(module: BFTaskModule, x: torch.Tensor) -> torch.Tensor:
    """Arg-max class of the clean network output at ``x`` (fp64 forward)."""
    params = module.params
    h = x.double()
    for op in module.get_entry_task().ops:
        if op.op_type == "linear":
            h = h.reshape(h.shape[0], -1) @ params[op.inputs[1]].double().t() + params[op.inputs[2]].double()
        elif op.op_type == "conv2d":
            h = torch.nn.functional.conv2d(h, params[op.inputs[1]].double(), params[op.inputs[2]].double(),
                                           stride=op.attrs.get("stride", 1), padding=op.attrs.get("padding", 0))
        elif op.op_type == "relu":
            h = h.clamp_min(0)
        elif op.op_type == "flatten":
            h = h.reshape(h.shape[0], -1)
    return h.argmax(dim=1)


def make_c1(seed: int = 0, batch: int = 64, eps: float = 2.0 / 255.0, label_mode: str = "random") -> Workload:
    """``label_mode="predicted"`` labels each input with the network's own
    prediction, which gives a mix of certified and uncertified inputs at small eps."""
    g = torch.Generator().manual_seed(seed)
    module = build_mlp([784, 256, 256, 10], gen=g)
    x = torch.rand(batch, 784, generator=g)
    labels = torch.randint(0, 10, (batch,), generator=g)
    if label_mode == "predicted":
        labels = predicted_labels(module, x)
    lo = torch.clamp(x - eps, 0.0, 1.0)
    hi = torch.clamp(x + eps, 0.0, 1.0)
    spec = InputSpec.box(value_name="input", lower=lo, upper=hi)
    return Workload("C1", module, spec, margin_spec(labels), labels)


def make_c2(seed: int = 0, batch: int = 256, width: int = 500, depth: int = 6) -> Workload:
    g = torch.Generator().manual_seed(seed)
    module = build_mlp([784] + [width] * depth + [10], gen=g, init="normal", bias_std=0.01)
    x = torch.rand(batch, 784, generator=g)
    labels = torch.randint(0, 10, (batch,), generator=g)
    spec = InputSpec.linf(value_name="input", center=x, eps=0.015)
    return Workload("C2", module, spec, margin_spec(labels), labels)


def make_c3(seed: int = 0, batch: int = 128, eps: float = 2.0 / 255.0, name: str = "C3") -> Workload:
    g = torch.Generator().manual_seed(seed)
    module = build_cnn(gen=g)
    x = torch.rand(batch, 3, 32, 32, generator=g)
    labels = torch.randint(0, 10, (batch,), generator=g)
    spec = InputSpec.linf(value_name="input", center=x, eps=eps)
    return Workload(name, module, spec, margin_spec(labels), labels)


def make_c4(seed: int = 0, batch: int = 32) -> Workload:
    w = make_c3(seed=seed, batch=batch, eps=8.0 / 255.0, name="C4")
    w.extra.update({"steps": 20, "lr": 0.1, "alpha_init": "crown"})
    return w


def make_dag(kind: str = "residual_mlp", seed: int = 0, batch: int = 8, eps: float = 0.02, box: bool = False,
             n_in: int = 16, hidden: int = 24, n_out: int = 10, channels: Tuple[int, int, int] = (2, 6, 6),
             blocks: int = 1, width: Optional[int] = None) -> Workload:
    """A DAG network of ``build_dag`` with a margin spec of random labels; the input
    set is a Linf ball of radius eps, or (box) that ball clamped to [0, 1]."""
    g = torch.Generator().manual_seed(seed)
    module = build_dag(kind, gen=g, n_in=n_in, hidden=hidden, n_out=n_out, channels=channels, blocks=blocks,
                       width=width)
    x = torch.rand((batch,) + dag_input_shape(kind, n_in=n_in, channels=channels), generator=g)
    labels = torch.randint(0, n_out, (batch,), generator=g)
    if box:
        spec = InputSpec.box(value_name="input", lower=torch.clamp(x - eps, 0.0, 1.0),
                             upper=torch.clamp(x + eps, 0.0, 1.0))
    else:
        spec = InputSpec.linf(value_name="input", center=x, eps=eps)
    return Workload(f"dag_{kind}", module, spec, margin_spec(labels, n_out), labels)


def _ibp_relu_bounds_f64(module: BFTaskModule, x: torch.Tensor, eps: float) -> List[Tuple[torch.Tensor, torch.Tensor]]:
    """Root pre-activation boxes of an MLP, fp64, used only to pick split candidates."""
    params = module.params
    ops = module.get_entry_task().ops
    l = (x - eps).double()
    u = (x + eps).double()
    out = []
    for op in ops:
        if op.op_type == "linear":
            W = params[op.inputs[1]].double()
            b = params[op.inputs[2]].double()
            c = (l + u) / 2
            r = (u - l) / 2
            mid = c @ W.t() + b
            rad = r @ W.abs().t()
            l, u = mid - rad, mid + rad
        elif op.op_type == "relu":
            out.append((l.clone(), u.clone()))
            l, u = l.clamp_min(0), u.clamp_min(0)
    return out


def make_c5(seed: int = 0, domains: int = 4096, eps: float = 0.03, max_splits: int = 12,
            width: int = 256, depth: int = 4, label_mode: str = "random") -> Workload:
    g = torch.Generator().manual_seed(seed)
    module = build_mlp([784] + [width] * depth + [10], gen=g)
    x0 = torch.rand(1, 784, generator=g)
    label = torch.randint(0, 10, (1,), generator=g)
    if label_mode == "predicted":
        label = predicted_labels(module, x0)
    relu_names = [op.inputs[0] for op in module.get_entry_task().ops if op.op_type == "relu"]
    root = _ibp_relu_bounds_f64(module, x0, eps)
    cand: List[Tuple[int, int]] = []
    for li, (l, u) in enumerate(root):
        amb = ((l[0] < 0) & (u[0] > 0)).nonzero(as_tuple=False).flatten().tolist()
        cand.extend((li, j) for j in amb)
    splits = {name: torch.zeros(domains, width, dtype=torch.int8) for name in relu_names}
    ncand = len(cand)
    for d in range(domains):
        k = int(torch.randint(1, max_splits + 1, (1,), generator=g))
        k = min(k, ncand)
        pick = torch.randperm(ncand, generator=g)[:k].tolist()
        signs = torch.randint(0, 2, (k,), generator=g) * 2 - 1
        for p, s in zip(pick, signs.tolist()):
            li, j = cand[p]
            splits[relu_names[li]][d, j] = int(s)
    x = x0.expand(domains, 784).contiguous()
    labels = label.expand(domains).contiguous()
    spec = InputSpec.linf(value_name="input", center=x, eps=eps)
    w = Workload("C5", module, spec, margin_spec(labels), labels)
    w.extra.update({"splits": splits, "steps": 10, "lr": 0.2, "alpha_init": 0.5, "beta_init": 0.0,
                    "num_candidates": ncand})
    return w


def make_ibp_dag(seed: int = 0, batch: int = 8, eps: float = 0.05, box: bool = False) -> Workload:
    """One-task IBP program that uses every op of the task executors: linear on
    the input set with a shared [O, I] and a per-sample [B, O, I] weight, relu,
    add, mul (by a mixed-sign gate), reshape, permute, flatten, concat and
    spec_linear.  Output value ``margins`` [B, 9]."""
    g = torch.Generator().manual_seed(1000 + seed)
    B = batch
    p: Dict[str, torch.Tensor] = {}
    p["W0"] = _kaiming((32, 24), fan_in=24, gen=g, kind="uniform")
    p["b0"] = torch.randn(32, generator=g) * 0.1
    p["W1"] = _kaiming((16, 32), fan_in=32, gen=g, kind="uniform")
    p["b1"] = torch.randn(16, generator=g) * 0.1
    p["W2"] = _kaiming((16, 32), fan_in=32, gen=g, kind="uniform")
    p["gate"] = torch.randn(16, generator=g)
    p["Wi"] = torch.randn(B, 8, 24, generator=g) * 0.2
    p["bi"] = torch.randn(B, 8, generator=g) * 0.1
    p["W3"] = _kaiming((10, 56), fan_in=56, gen=g, kind="uniform")
    p["b3"] = torch.randn(10, generator=g) * 0.1
    x = torch.rand(B, 24, generator=g)
    labels = torch.randint(0, 10, (B,), generator=g)
    p["C"] = margin_spec(labels)
    ops = [
        TaskOp("linear", "linear0", ["input", "W0", "b0"], ["h0"]),
        TaskOp("relu", "relu0", ["h0"], ["r0"]),
        TaskOp("linear", "linear1", ["r0", "W1", "b1"], ["a"]),
        TaskOp("linear", "linear2", ["r0", "W2"], ["c"]),
        TaskOp("add", "add", ["a", "c"], ["s"]),
        TaskOp("mul", "mul", ["s", "gate"], ["m"]),
        TaskOp("reshape", "reshape", ["r0"], ["rr"], {"shape": [B, 2, 16]}),
        TaskOp("permute", "permute", ["rr"], ["rp"], {"dims": [0, 2, 1]}),
        TaskOp("flatten", "flatten", ["rp"], ["rf"], {"start_dim": 1, "end_dim": -1}),
        TaskOp("linear", "linear_in", ["input", "Wi", "bi"], ["hi"]),
        TaskOp("concat", "concat", ["m", "rf", "hi"], ["cat"], {"axis": 1}),
        TaskOp("relu", "relu1", ["cat"], ["rc"]),
        TaskOp("linear", "linear3", ["rc", "W3", "b3"], ["out"]),
        TaskOp("spec_linear", "spec", ["out", "C"], ["margins"]),
    ]
    values = ["input", "h0", "r0", "a", "c", "s", "m", "rr", "rp", "rf", "hi", "cat", "rc", "out", "margins"]
    task = BoundTask(task_id="t0", kind=TaskKind.INTERVAL_IBP, ops=ops, input_values=["input"],
                     output_values=["margins"], params=list(p.keys()))
    module = BFTaskModule(tasks=[task], entry_task_id="t0", bindings={"params": p},
                          storage_plan=default_storage_plan(values))
    if box:
        spec = InputSpec.box(value_name="input", lower=torch.clamp(x - eps, 0.0, 1.0),
                             upper=torch.clamp(x + eps, 0.0, 1.0))
    else:
        spec = InputSpec.linf(value_name="input", center=x, eps=eps)
    return Workload("ibp_dag", module, spec, p["C"], labels)


def make_bab_toy(seed: int = 0, batch: int = 6, eps: float = 0.08, dims: Sequence[int] = (12, 16, 16, 4)) -> Workload:
    """Small MLP for whole branch-and-bound searches: inputs in [0, 1]^12, Linf
    eps, margin specs of the network's own prediction (so some examples are
    provable, some are not)."""
    g = torch.Generator().manual_seed(2000 + seed)
    module = build_mlp(list(dims), gen=g, bias_std=0.1)
    x = torch.rand(batch, dims[0], generator=g)
    labels = predicted_labels(module, x)
    spec = InputSpec.linf(value_name="input", center=x, eps=eps)
    return Workload("bab_toy", module, spec, margin_spec(labels, dims[-1]), labels)


def build_small_cnn(*, gen: torch.Generator, in_shape: Sequence[int] = (2, 6, 6), channels: int = 4,
                    kernel: int = 3, stride: int = 1, padding: int = 0, hidden: int = 10, n_out: int = 3,
                    bias_std: float = 0.1, conv_bias_std: float = 0.1) -> BFTaskModule:
    """in_shape -> conv(channels, kernel, stride, padding) -> relu -> flatten -> fc hidden -> relu -> fc n_out."""
    ci, hi, wi = (int(d) for d in in_shape)
    ho = (hi + 2 * padding - kernel) // stride + 1
    wo = (wi + 2 * padding - kernel) // stride + 1
    n_flat = channels * ho * wo
    params: Dict[str, torch.Tensor] = {
        "W0": _kaiming((channels, ci, kernel, kernel), fan_in=ci * kernel * kernel, gen=gen, kind="uniform"),
        "b0": _bias(channels, gen, conv_bias_std),
        "W1": _kaiming((hidden, n_flat), fan_in=n_flat, gen=gen, kind="uniform"),
        "b1": _bias(hidden, gen, bias_std),
        "W2": _kaiming((n_out, hidden), fan_in=hidden, gen=gen, kind="uniform"),
        "b2": _bias(n_out, gen, bias_std),
    }
    conv = {"stride": stride, "padding": padding, "dilation": 1, "groups": 1}
    ops = [TaskOp("conv2d", "conv0", ["input", "W0", "b0"], ["h0"], conv),
           TaskOp("relu", "relu0", ["h0"], ["r0"]),
           TaskOp("flatten", "flatten", ["r0"], ["f0"], {"start_dim": 1, "end_dim": -1}),
           TaskOp("linear", "linear1", ["f0", "W1", "b1"], ["h1"]),
           TaskOp("relu", "relu1", ["h1"], ["r1"]),
           TaskOp("linear", "linear2", ["r1", "W2", "b2"], ["out"])]
    return _module(ops, params, ["input", "h0", "r0", "f0", "h1", "r1", "out"])


def make_bab_cnn_toy(seed: int = 0, batch: int = 4, eps: float = 0.02, in_shape: Sequence[int] = (2, 6, 6),
                     channels: int = 4, hidden: int = 10, n_out: int = 3, conv_bias_std: float = 0.1) -> Workload:
    """Small CNN for whole branch-and-bound searches on conv graphs: inputs in
    [0, 1]^in_shape, Linf eps, margin specs of the network's own prediction."""
    g = torch.Generator().manual_seed(3000 + seed)
    module = build_small_cnn(gen=g, in_shape=in_shape, channels=channels, hidden=hidden, n_out=n_out,
                             conv_bias_std=conv_bias_std)
    x = torch.rand((batch,) + tuple(int(d) for d in in_shape), generator=g)
    labels = predicted_labels(module, x)
    spec = InputSpec.linf(value_name="input", center=x, eps=eps)
    return Workload("bab_cnn_toy", module, spec, margin_spec(labels, n_out), labels)


def make_wide_cnn(seed: int = 0, batch: int = 4, eps: float = 2.0 / 255.0) -> Workload:
    """A CNN whose first conv writes a 32x32x32 map (128 KB per row, beyond a 64 KB LDS
    row stage): 3x32x32 -> conv(32, 3x3, s1, p1) -> relu -> conv(16, 4x4, s2, p1)
    16x16x16 -> relu -> flatten -> fc 4096 -> 10; Kaiming-uniform weights, small
    biases, inputs uniform in [0, 1], Linf eps, 9 margin specs of random labels."""
    g = torch.Generator().manual_seed(4000 + seed)
    params: Dict[str, torch.Tensor] = {
        "W0": _kaiming((32, 3, 3, 3), fan_in=27, gen=g, kind="uniform"), "b0": _bias(32, g, 0.05),
        "W1": _kaiming((16, 32, 4, 4), fan_in=512, gen=g, kind="uniform"), "b1": _bias(16, g, 0.05),
        "W2": _kaiming((10, 4096), fan_in=4096, gen=g, kind="uniform"), "b2": _bias(10, g, 0.05),
    }
    ops = [TaskOp("conv2d", "conv0", ["input", "W0", "b0"], ["h0"], {"stride": 1, "padding": 1, "dilation": 1,
                                                                     "groups": 1}),
           TaskOp("relu", "relu0", ["h0"], ["r0"]),
           TaskOp("conv2d", "conv1", ["r0", "W1", "b1"], ["h1"], {"stride": 2, "padding": 1, "dilation": 1,
                                                                  "groups": 1}),
           TaskOp("relu", "relu1", ["h1"], ["r1"]),
           TaskOp("flatten", "flatten", ["r1"], ["f1"], {"start_dim": 1, "end_dim": -1}),
           TaskOp("linear", "linear2", ["f1", "W2", "b2"], ["out"])]
    module = _module(ops, params, ["input", "h0", "r0", "h1", "r1", "f1", "out"])
    x = torch.rand(batch, 3, 32, 32, generator=g)
    labels = torch.randint(0, 10, (batch,), generator=g)
    spec = InputSpec.linf(value_name="input", center=x, eps=eps)
    return Workload("wide_cnn", module, spec, margin_spec(labels), labels)


def make_bab_case(kind: str = "mlp", **kw) -> Workload:
    """The whole-search workloads: ``make_bab_toy`` (kind "mlp") or ``make_bab_cnn_toy`` (kind "cnn")."""
    return make_bab_cnn_toy(**kw) if kind == "cnn" else make_bab_toy(**kw)


def split_ibp_dag(w: Workload) -> BFTaskModule:
    """The ``make_ibp_dag`` program as three tasks joined by a TaskGraph, with a
    storage plan that reuses physical buffers (``h0``/``a`` and ``c``/``rr``
    share one each: the first of each pair is dead before the second is
    written)."""
    ops = {op.name: op for op in w.module.get_entry_task().ops}
    groups = {
        "t0": (["linear0", "relu0"], ["input"], ["r0"]),
        "t1": (["linear1", "linear2", "add", "mul", "reshape", "permute", "flatten", "linear_in"],
               ["r0", "input"], ["m", "rf", "hi"]),
        "t2": (["concat", "relu1", "linear3", "spec"], ["m", "rf", "hi"], ["margins"]),
    }
    # ``gate`` is a parameter read as an interval operand (mul); run_ibp_task
    # resolves such operands through the storage plan as well
    values = ["input", "h0", "r0", "a", "c", "s", "gate", "m", "rr", "rp", "rf", "hi", "cat", "rc", "out",
              "margins"]
    plan = StoragePlan()
    for v in values:
        plan.buffers[f"buf_{v}"] = BufferSpec(buffer_id=f"buf_{v}", dtype="float32", shape=[None])
        plan.value_to_buffer[v] = f"buf_{v}"
    alias = {"buf_a": "phys_h0_a", "buf_h0": "phys_h0_a", "buf_c": "phys_c_rr", "buf_rr": "phys_c_rr"}
    for lb in plan.buffers:
        pb = alias.get(lb, "phys_" + lb[4:])
        plan.logical_to_physical[lb] = pb
        plan.physical_buffers[pb] = BufferSpec(buffer_id=pb, dtype="float32", shape=[None])
    tasks = []
    for tid, (names, ins, outs) in groups.items():
        tasks.append(BoundTask(task_id=tid, kind=TaskKind.INTERVAL_IBP, ops=[ops[n] for n in names],
                               input_values=ins, output_values=outs,
                               input_buffers=[plan.value_to_buffer[v] for v in ins],
                               output_buffers=[plan.value_to_buffer[v] for v in outs]))

    def dep(v):
        return TaskBufferDep(src_value=v, src_buffer_id=plan.value_to_buffer[v], dst_value=v,
                             dst_buffer_id=plan.value_to_buffer[v])

    graph = TaskGraph(task_ids=["t0", "t1", "t2"], edges=[
        TaskDepEdge(src_task_id="t0", dst_task_id="t1", deps=[dep("r0")]),
        TaskDepEdge(src_task_id="t1", dst_task_id="t2", deps=[dep("m"), dep("rf"), dep("hi")]),
    ])
    return BFTaskModule(tasks=tasks, entry_task_id="t0", bindings={"params": w.module.params}, storage_plan=plan,
                        task_graph=graph)


def make_d1(seed: int = 0, batch: int = 256, eps: float = 0.002) -> Workload:
    """D1: CROWN on a residual MLP, 784 -> 256 stem, 4 blocks 256-512-256 with identity
    skips, head 10; B=256, Linf eps, 9 margin specs."""
    w = make_dag("residual_mlp", seed=seed, batch=batch, eps=eps, n_in=784, hidden=512, width=256, blocks=4)
    w.name = "D1"
    return w


MAKERS = {"C1": make_c1, "C2": make_c2, "C3": make_c3, "C4": make_c4, "C5": make_c5, "D1": make_d1}


def make(name: str, **kw) -> Workload:
    return MAKERS[name](**kw)


def relu_input_names(module: BFTaskModule) -> List[str]:
    return [op.inputs[0] for op in module.get_entry_task().ops if op.op_type == "relu"]


def to_device(w: Workload, device) -> Workload:
    """Copy a workload (params, spec, C, splits) to ``device``."""
    params = {k: v.to(device) for k, v in w.module.params.items()}
    mod = BFTaskModule(tasks=w.module.tasks, entry_task_id=w.module.entry_task_id,
                       bindings={"params": params}, storage_plan=w.module.storage_plan,
                       task_graph=w.module.task_graph)
    extra = dict(w.extra)
    if "splits" in extra:
        extra["splits"] = {k: v.to(device) for k, v in extra["splits"].items()}
    return Workload(w.name, mod, w.spec.to(device), w.C.to(device), w.labels.to(device), extra)


def subset(w: Workload, n: int) -> Workload:
    """First ``n`` inputs/domains of a workload (same network)."""
    spec = w.spec
    if hasattr(spec.perturbation, "lower"):
        spec = InputSpec.box(value_name=spec.value_name, lower=spec.perturbation.lower[:n],
                             upper=spec.perturbation.upper[:n])
    else:
        spec = InputSpec(value_name=spec.value_name, center=spec.center[:n], perturbation=spec.perturbation)
    extra = dict(w.extra)
    if "splits" in extra:
        extra["splits"] = {k: v[:n] for k, v in extra["splits"].items()}
    return Workload(w.name, w.module, spec, w.C[:n], w.labels[:n], extra)
