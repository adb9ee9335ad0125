"""Pin the IBP task-executor oracle (oracle/task_ibp_ref.py).

* against fixtures written by the reference's PythonTaskExecutor.run_ibp and
  run_ibp_scheduled (tests/golden/make_golden.py);
* by what the mathematics fixes: every sampled point of the input set maps
  inside the bounds (soundness); one affine layer on an Linf ball is exact, its
  bound attained at the vertex ``x0 + eps * sign(w)``; the interval product
  equals the brute-force min/max over the four corners; the scheduled run over
  the three-task split equals the one-task run.
"""

import pytest
import torch

from boundflow_amd import workloads as wl
from boundflow_amd.ir import BFTaskModule, BoundTask, TaskKind, TaskOp, default_storage_plan
from boundflow_amd.spec import InputSpec, IntervalState
from oracle import task_ibp_ref as ti
from tests.golden_util import load, t, workload_checksum


def _close(a, b, rtol=1e-6, atol=1e-6):
    a = torch.as_tensor(a).double()
    b = torch.as_tensor(b).double()
    assert a.shape == b.shape, (tuple(a.shape), tuple(b.shape))
    assert torch.allclose(a, b, rtol=rtol, atol=atol), float((a - b).abs().max())


CASES = [
    ("task_ibp_c1_b8", lambda: wl.subset(wl.make_c1(), 8)),
    ("task_ibp_c3_b4", lambda: wl.subset(wl.make_c3(), 4)),
    ("task_ibp_dag", lambda: wl.make_ibp_dag()),
    ("task_ibp_dag_box", lambda: wl.make_ibp_dag(box=True)),
]


@pytest.mark.parametrize("tag,maker", CASES)
def test_run_ibp_matches_reference(tag, maker):
    g = load(tag)
    w = maker()
    assert workload_checksum(w) == str(g["checksum"]), "workload generator drifted from the fixture"
    out = ti.run_ibp(w.module, w.spec)
    _close(out.lower, g["lower"])
    _close(out.upper, g["upper"])


def test_run_ibp_scheduled_matches_reference():
    g = load("task_ibp_dag_sched")
    w = wl.make_ibp_dag()
    assert workload_checksum(w) == str(g["checksum"])
    out = ti.run_ibp_scheduled(wl.split_ibp_dag(w), w.spec)
    _close(out.lower, g["lower"])
    _close(out.upper, g["upper"])


def test_scheduled_equals_single_task():
    """Same program, same input box: only the first layer's association differs
    (interval W+/W- on x0 -+ eps against concretize_matmul)."""
    w = wl.make_ibp_dag()
    one = ti.run_ibp(w.module, w.spec)
    many = ti.run_ibp_scheduled(wl.split_ibp_dag(w), w.spec)
    _close(one.lower, many.lower, rtol=1e-5, atol=1e-5)
    _close(one.upper, many.upper, rtol=1e-5, atol=1e-5)


def _concrete(module: BFTaskModule, x: torch.Tensor) -> torch.Tensor:
    """Plain fp64 evaluation of the program at one batch of points."""
    p = {k: v.double() for k, v in module.params.items()}
    env = {"input": x.double()}
    for op in module.get_entry_task().ops:
        a = [env[n] if n in env else p[n] for n in op.inputs]
        k = op.op_type
        if k == "linear":
            W = a[1]
            y = torch.bmm(a[0].unsqueeze(1), W.transpose(1, 2)).squeeze(1) if W.dim() == 3 else a[0] @ W.t()
            env[op.outputs[0]] = y + a[2] if len(a) == 3 else y
        elif k == "conv2d":
            env[op.outputs[0]] = torch.nn.functional.conv2d(a[0], a[1], a[2], stride=op.attrs["stride"],
                                                            padding=op.attrs["padding"])
        elif k == "relu":
            env[op.outputs[0]] = a[0].clamp_min(0)
        elif k == "add":
            env[op.outputs[0]] = a[0] + a[1]
        elif k == "mul":
            env[op.outputs[0]] = a[0] * a[1]
        elif k == "reshape":
            env[op.outputs[0]] = a[0].reshape(op.attrs["shape"])
        elif k == "permute":
            env[op.outputs[0]] = a[0].permute(*op.attrs["dims"])
        elif k == "flatten":
            env[op.outputs[0]] = torch.flatten(a[0], op.attrs.get("start_dim", 0), op.attrs.get("end_dim", -1))
        elif k == "concat":
            env[op.outputs[0]] = torch.cat(a, dim=1)
        elif k == "spec_linear":
            env[op.outputs[0]] = torch.bmm(a[1], a[0].unsqueeze(-1)).squeeze(-1)
        else:
            raise AssertionError(k)
    return env[module.get_entry_task().output_values[0]]


@pytest.mark.parametrize("box", [False, True])
def test_dag_bounds_are_sound(box):
    w = wl.make_ibp_dag(box=box)
    out = ti.run_ibp(w.module, w.spec)
    g = torch.Generator().manual_seed(3)
    lo, hi = w.spec.perturbation.bounding_box(w.spec.center)
    for _ in range(64):
        r = torch.rand(lo.shape, generator=g, dtype=torch.float64)
        r = torch.where(r < 0.25, torch.zeros_like(r), torch.where(r > 0.75, torch.ones_like(r), r))
        x = lo.double() + r * (hi - lo).double()
        y = _concrete(w.module, x)
        assert bool((y >= out.lower.double() - 1e-5).all()) and bool((y <= out.upper.double() + 1e-5).all())


def test_single_affine_layer_is_exact():
    g = torch.Generator().manual_seed(4)
    W = torch.randn(7, 12, generator=g)
    b = torch.randn(7, generator=g)
    x0 = torch.rand(3, 12, generator=g)
    eps = 0.1
    op = TaskOp("linear", "l", ["input", "W", "b"], ["out"])
    task = BoundTask(task_id="t", kind=TaskKind.INTERVAL_IBP, ops=[op], input_values=["input"],
                     output_values=["out"])
    m = BFTaskModule(tasks=[task], entry_task_id="t", bindings={"params": {"W": W, "b": b}},
                     storage_plan=default_storage_plan(["input", "out"]))
    out = ti.run_ibp(m, InputSpec.linf(value_name="input", center=x0, eps=eps))
    Wd = W.double()
    top = ((x0.double().unsqueeze(1) + eps * Wd.sign().unsqueeze(0)) * Wd.unsqueeze(0)).sum(-1) + b.double()
    bot = ((x0.double().unsqueeze(1) - eps * Wd.sign().unsqueeze(0)) * Wd.unsqueeze(0)).sum(-1) + b.double()
    _close(out.upper, top, rtol=1e-5, atol=1e-5)
    _close(out.lower, bot, rtol=1e-5, atol=1e-5)


def test_interval_mul_is_corner_min_max():
    g = torch.Generator().manual_seed(5)
    al = torch.randn(200, generator=g)
    au = al + torch.rand(200, generator=g) * 2
    bl = torch.randn(200, generator=g)
    bu = bl + torch.rand(200, generator=g) * 2
    op = TaskOp("mul", "m", ["a", "b"], ["c"])
    env = {"a": IntervalState(al, au), "b": IntervalState(bl, bu)}
    out = ti._apply(op, lambda n: env[n], None)
    # brute force on a grid of each box: products are bilinear, extremes lie on corners
    s = torch.linspace(0, 1, 11, dtype=torch.float64)
    xa = al.double()[:, None] + s[None, :] * (au - al).double()[:, None]
    xb = bl.double()[:, None] + s[None, :] * (bu - bl).double()[:, None]
    prod = xa[:, :, None] * xb[:, None, :]
    _close(out.lower, prod.amin(dim=(1, 2)), rtol=1e-6, atol=1e-6)
    _close(out.upper, prod.amax(dim=(1, 2)), rtol=1e-6, atol=1e-6)
