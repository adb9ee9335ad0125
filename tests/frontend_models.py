"""``torch.nn.Module`` versions of the seeded benchmark networks (test
infrastructure): the same weights as the hand-built task modules of
``boundflow_amd.workloads``, so that importing them through the PyTorch
frontend and planner v0 must give the same bounds bit for bit."""

import numpy as np  # noqa: F401
import torch
import torch.nn as nn


def sequential_from_chain(module) -> nn.Sequential:
    """nn.Sequential of a chain task module (linear / conv2d / relu / flatten ops)."""
    params = module.params
    layers = []
    for op in module.get_entry_task().ops:
        if op.op_type == "linear":
            W, b = params[op.inputs[1]], params[op.inputs[2]]
            lin = nn.Linear(int(W.shape[1]), int(W.shape[0]))
            with torch.no_grad():
                lin.weight.copy_(W)
                lin.bias.copy_(b)
            layers.append(lin)
        elif op.op_type == "conv2d":
            W, b = params[op.inputs[1]], params[op.inputs[2]]
            a = op.attrs
            conv = nn.Conv2d(int(W.shape[1]), int(W.shape[0]), tuple(W.shape[2:]), stride=a.get("stride", 1),
                             padding=a.get("padding", 0))
            with torch.no_grad():
                conv.weight.copy_(W)
                conv.bias.copy_(b)
            layers.append(conv)
        elif op.op_type == "relu":
            layers.append(nn.ReLU())
        elif op.op_type == "flatten":
            layers.append(nn.Flatten(op.attrs.get("start_dim", 1), op.attrs.get("end_dim", -1)))
        else:
            raise NotImplementedError(op.op_type)
    return nn.Sequential(*layers).eval()


class ResidualAddNet(nn.Module):
    """The reference's general-DAG frontend test network (tests/test_phase7a_pr8_general_dag_frontends.py:37-48)."""

    def __init__(self) -> None:
        super().__init__()
        self.main = nn.Conv2d(1, 2, 1)
        self.skip = nn.Conv2d(1, 2, 1)
        self.head = nn.Linear(8, 3)

    def forward(self, x):
        main = torch.relu(self.main(x))
        skip = self.skip(x)
        out = torch.relu(main + skip)
        return self.head(out.flatten(1))


class ConcatNet(nn.Module):
    """tests/test_phase7a_pr8_general_dag_frontends.py:51-63 of the reference."""

    def __init__(self) -> None:
        super().__init__()
        self.left = nn.Conv2d(1, 2, 1)
        self.right = nn.Conv2d(1, 1, 1)
        self.head = nn.Linear(12, 4)

    def forward(self, x):
        left = torch.relu(self.left(x))
        right = torch.relu(self.right(x))
        cat = torch.cat([left, right], dim=1)
        return self.head(cat.flatten(1))


class PermuteNet(nn.Module):
    """Layout-only permutes (composed to identity, and one kept) for the planner pass."""

    def __init__(self) -> None:
        super().__init__()
        self.fc = nn.Linear(6, 3)

    def forward(self, x):
        y = x.permute(0, 2, 1).permute(0, 2, 1)      # composes to the identity
        z = y.permute(0, 2, 1)
        return self.fc(z.reshape(z.shape[0], 6))


def seeded(cls, seed: int = 0):
    torch.manual_seed(seed)
    return cls().eval()


def planned_module_json(tm) -> str:
    """The fields of a planned task module the HIP backend reads, as canonical JSON."""
    import json
    task = tm.get_entry_task()
    sp = tm.storage_plan

    def conv(v):
        if isinstance(v, (list, tuple)):
            return [conv(x) for x in v]
        if isinstance(v, dict):
            return {k: conv(x) for k, x in v.items()}
        return v

    out = {
        "task": {"task_id": task.task_id, "kind": task.kind.value, "input_values": list(task.input_values),
                 "output_values": list(task.output_values), "input_buffers": list(task.input_buffers),
                 "output_buffers": list(task.output_buffers), "params": list(task.params),
                 "lowering": task.lowering.value},
        "ops": [{"op_type": o.op_type, "name": o.name, "inputs": list(o.inputs), "outputs": list(o.outputs),
                 "attrs": conv(dict(o.attrs))} for o in task.ops],
        "buffers": {k: {"dtype": b.dtype, "shape": list(b.shape), "scope": b.scope, "device": b.device,
                        "layout": b.layout} for k, b in sp.buffers.items()},
        "value_to_buffer": dict(sp.value_to_buffer),
        "param_shapes": {k: list(v.shape) for k, v in tm.bindings["params"].items()},
    }
    return json.dumps(out, sort_keys=True)


def frontend_nets():
    """name -> (nn.Module, example input) of the frontend fixtures."""
    from boundflow_amd import workloads as wl
    c1 = wl.subset(wl.make_c1(), 4)
    c3 = wl.subset(wl.make_c3(), 4)
    g = torch.Generator().manual_seed(3)
    return {
        "c1_mlp": (sequential_from_chain(c1.module), c1.spec.perturbation.lower),
        "c3_cnn": (sequential_from_chain(c3.module), c3.spec.center),
        "residual_add": (seeded(ResidualAddNet), torch.rand(2, 1, 2, 2, generator=g)),
        "concat": (seeded(ConcatNet), torch.rand(2, 1, 2, 2, generator=g)),
        "permute": (seeded(PermuteNet), torch.rand(2, 3, 2, generator=g)),
    }


VNNLIB_SOURCES = {
    "reference_example": (
        "; compact classification property\n(declare-const X_0 Real)\n(declare-const X_1 Real)\n"
        "(declare-const Y_0 Real)\n(declare-const Y_1 Real)\n(declare-const Y_2 Real)\n"
        "(assert (>= X_0 -1.0))\n(assert (<= X_0 2.0))\n(assert (<= 0.25 X_1))\n(assert (>= 3.5 X_1))\n"
        "(assert (or\n  (and (>= Y_0 Y_2))\n  (and (<= Y_1 Y_2))\n))\n"),
    "linear_terms": (
        "(declare-const X_0 Real)\n(declare-const Y_0 Real)\n(declare-const Y_1 Real)\n"
        "(assert (<= X_0 0.5))\n(assert (>= X_0 -0.5))\n"
        "(assert (or (and (>= (+ Y_0 1.5) (* 2.0 Y_1))) (< (- Y_1 Y_0 0.25) (* Y_0 -3))\n"
        "  (> 1e-3 (- Y_1)) (<= (* 0.5 (+ Y_0 Y_1)) -2)))\n"),
}


def vnnlib_c1_property(index: int = 0) -> str:
    """A VNN-COMP style robustness property of C1's input ``index``: its clamped
    2/255 box, unsafe if some other class scores at least the label's."""
    from boundflow_amd import workloads as wl
    w = wl.make_c1()
    lo, hi = w.spec.perturbation.lower[index], w.spec.perturbation.upper[index]
    y = int(w.labels[index])
    lines = [f"(declare-const X_{i} Real)" for i in range(784)] + [f"(declare-const Y_{j} Real)" for j in range(10)]
    for i in range(784):
        lines.append(f"(assert (>= X_{i} {float(lo[i])!r}))")
        lines.append(f"(assert (<= X_{i} {float(hi[i])!r}))")
    lines.append("(assert (or " + " ".join(f"(and (>= Y_{j} Y_{y}))" for j in range(10) if j != y) + "))")
    return "\n".join(lines) + "\n"




def native_toy():
    """The reference's native-queue toy (tests/test_native_relu_split_bab_runtime.py:20-56)."""
    from boundflow_amd.ir import BFTaskModule, BoundTask, TaskKind, TaskOp
    from boundflow_amd.spec import InputSpec
    ops = [TaskOp("linear", "linear1", ["input", "W1", "b1"], ["h1"]), TaskOp("relu", "relu1", ["h1"], ["r1"]),
           TaskOp("linear", "linear2", ["r1", "W2", "b2"], ["out"])]
    params = {"W1": torch.tensor([[1.0, -0.5, 0.25], [-0.25, 0.75, 1.0], [0.5, 0.5, -1.0]]),
              "b1": torch.tensor([0.1, -0.2, 0.05]),
              "W2": torch.tensor([[0.75, -1.0, 0.5], [-0.5, 0.25, 1.25]]), "b2": torch.tensor([0.15, -0.1])}
    task = BoundTask(task_id="native-relu-split-toy", kind=TaskKind.INTERVAL_IBP, ops=ops, input_values=["input"],
                     output_values=["out"])
    module = BFTaskModule(tasks=[task], entry_task_id=task.task_id, bindings={"params": params})
    spec = InputSpec.box(value_name="input", lower=torch.tensor([[-0.3, -0.6, -0.1]]),
                         upper=torch.tensor([[0.7, 0.4, 0.9]]))
    return module, spec, torch.tensor([[1.0, -1.0]])


def native_bab_toy():
    """A four-layer MLP (make_bab_toy's, seed 1, 6-12-12-3) on a box, objective y_0 - y_1."""
    from boundflow_amd.spec import InputSpec
    from boundflow_amd import workloads as wl
    w = wl.make_bab_toy(seed=1, eps=0.2, dims=(6, 12, 12, 3), batch=1)
    x = w.spec.center
    spec = InputSpec.box(value_name="input", lower=x - 0.2, upper=x + 0.2)
    return w.module, spec, torch.tensor([[1.0, -1.0, 0.0]])


