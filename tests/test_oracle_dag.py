"""Pin the oracle's CROWN backward on DAG networks (fan-in accumulation, add and
concat adjoints, crown_ibp.py:874-937 and 1928-2030) without the reference.

* soundness: the bounds of the four reference DAG shapes contain the network's
  value at sampled points of the input set;
* exactness: with every ReLU stable the network is affine on the input set, and
  CROWN's bounds equal f(x0) -/+ eps * |J| 1 (Linf) or f(mid) -/+ |J| rad (box)
  with J the Jacobian from autograd -- a dropped branch, a bias counted twice or
  a slice taken from the wrong columns fails this;
* equivalence: a value read by two linear layers whose outputs are added bounds
  exactly like the chain with the summed weight (the relaxation sees the
  accumulated coefficient), and a concat of two linear (conv) outputs like the
  chain with the stacked weight (channels), at an eps with ambiguous ReLUs.
All in float64.
"""

import pytest
import torch
import torch.nn.functional as F

from boundflow_amd import workloads as wl
from boundflow_amd.ir import BFTaskModule, BoundTask, TaskKind, TaskOp
from boundflow_amd.spec import InputSpec
from oracle import crown_ref as cr


def _to64(module: BFTaskModule) -> BFTaskModule:
    task = module.get_entry_task()
    params = {k: v.to(torch.float64) for k, v in module.params.items()}
    return BFTaskModule(tasks=[task], entry_task_id=task.task_id, bindings={"params": params})


def _module(ops, params):
    task = BoundTask(task_id="t0", kind=TaskKind.INTERVAL_IBP, ops=ops, input_values=["input"],
                     output_values=["out"])
    return BFTaskModule(tasks=[task], entry_task_id="t0", bindings={"params": params})


def evaluate(module: BFTaskModule, x: torch.Tensor) -> torch.Tensor:
    """Concrete forward pass of a task (the network the bounds are about)."""
    env = {"input": x}
    params = module.params

    def get(name):
        return env[name] if name in env else params[name]

    for op in module.get_entry_task().ops:
        t = op.op_type
        if t == "linear":
            b = params[op.inputs[2]] if len(op.inputs) == 3 else None
            y = F.linear(get(op.inputs[0]), params[op.inputs[1]], b)
        elif t == "conv2d":
            b = params[op.inputs[2]] if len(op.inputs) == 3 else None
            y = F.conv2d(get(op.inputs[0]), params[op.inputs[1]], b, stride=op.attrs.get("stride", 1),
                         padding=op.attrs.get("padding", 0))
        elif t == "relu":
            y = torch.relu(get(op.inputs[0]))
        elif t == "add":
            y = get(op.inputs[0]) + get(op.inputs[1])
        elif t == "concat":
            y = torch.cat([get(n) for n in op.inputs], dim=int(op.attrs.get("axis", 1)))
        elif t == "flatten":
            y = torch.flatten(get(op.inputs[0]), 1)
        else:
            raise NotImplementedError(t)
        env[op.outputs[0]] = y
    return env[module.get_entry_task().output_values[0]]


def _case(kind, seed=0, batch=3, blocks=2):
    g = torch.Generator().manual_seed(seed)
    module = _to64(wl.build_dag(kind, gen=g, blocks=blocks))
    x = torch.rand((batch,) + wl.dag_input_shape(kind), generator=g, dtype=torch.float64)
    return module, x


def _ambiguous_count(relu_pre) -> int:
    return sum(int(((p.lower < 0) & (p.upper > 0)).sum()) for p in relu_pre.values())


@pytest.mark.parametrize("kind", wl.DAG_KINDS)
@pytest.mark.parametrize("box", [False, True])
def test_dag_bounds_contain_sampled_outputs(kind, box):
    module, x = _case(kind, seed=1)
    eps = 0.05
    if box:
        g = torch.Generator().manual_seed(7)
        rad = torch.rand(x.shape, generator=g, dtype=torch.float64) * eps
        spec = InputSpec.box(value_name="input", lower=x - rad, upper=x + rad)
        lo, hi = x - rad, x + rad
    else:
        spec = InputSpec.linf(value_name="input", center=x, eps=eps)
        lo, hi = x - eps, x + eps
    interval_env, relu_pre = cr.forward_ibp_trace(module, spec)
    assert _ambiguous_count(relu_pre) > 0
    out = cr.crown_backward_from_trace(module, spec, interval_env=interval_env, relu_pre=relu_pre)
    g = torch.Generator().manual_seed(11)
    n = 256
    u = torch.rand((n,) + tuple(x.shape), generator=g, dtype=torch.float64)
    u[: n // 2] = torch.round(u[: n // 2])          # vertices of the box
    pts = lo.unsqueeze(0) + u * (hi - lo).unsqueeze(0)
    ys = torch.stack([evaluate(module, p) for p in pts])
    assert bool((ys >= out.lower.unsqueeze(0) - 1e-9).all())
    assert bool((ys <= out.upper.unsqueeze(0) + 1e-9).all())
    # and CROWN is no looser than IBP's output box on these networks' spec rows by much:
    # at least one bound is strictly inside the sampled range's complement (not vacuous)
    assert bool(torch.isfinite(out.lower).all()) and bool(torch.isfinite(out.upper).all())


def _const_add_module(seed=3):
    """h = W1 x + b1 -> add(h, P) with a per-sample constant P [B, n] -> relu -> W2."""
    g = torch.Generator().manual_seed(seed)
    W1 = torch.randn(12, 6, generator=g, dtype=torch.float64)
    b1 = torch.randn(12, generator=g, dtype=torch.float64)
    P = torch.randn(2, 12, generator=g, dtype=torch.float64)
    W2 = torch.randn(5, 12, generator=g, dtype=torch.float64)
    ops = [TaskOp("linear", "lin1", ["input", "W1", "b1"], ["h"]),
           TaskOp("add", "add0", ["h", "P"], ["s"]),
           TaskOp("relu", "relu0", ["s"], ["r"]),
           TaskOp("linear", "lin2", ["r", "W2"], ["out"])]
    x = torch.rand(2, 6, generator=g, dtype=torch.float64)
    return _module(ops, {"W1": W1, "b1": b1, "P": P, "W2": W2}), x


@pytest.mark.parametrize("kind", list(wl.DAG_KINDS) + ["const_add"])
@pytest.mark.parametrize("box", [False, True])
def test_dag_bounds_exact_when_every_relu_is_stable(kind, box):
    if kind == "const_add":
        module, x = _const_add_module()
    else:
        module, x = _case(kind, seed=2, batch=2)
    eps = 1e-5
    if box:
        g = torch.Generator().manual_seed(5)
        rad = torch.rand(x.shape, generator=g, dtype=torch.float64) * eps
        spec = InputSpec.box(value_name="input", lower=x - rad, upper=x + rad)
    else:
        rad = torch.full_like(x, eps)
        spec = InputSpec.linf(value_name="input", center=x, eps=eps)
    interval_env, relu_pre = cr.forward_ibp_trace(module, spec)
    assert _ambiguous_count(relu_pre) == 0, "pick a smaller eps: some ReLU is unstable"
    out = cr.crown_backward_from_trace(module, spec, interval_env=interval_env, relu_pre=relu_pre)
    f = evaluate(module, x)
    Jall = torch.autograd.functional.jacobian(lambda z: evaluate(module, z), x)   # [B, out, B, *in]
    for b in range(int(x.shape[0])):
        f0 = f[b]
        J = Jall[b, :, b].reshape(int(f0.numel()), -1)
        dev = (J.abs() * rad[b].reshape(1, -1)).sum(dim=1)
        torch.testing.assert_close(out.lower[b], f0 - dev, rtol=0, atol=1e-10)
        torch.testing.assert_close(out.upper[b], f0 + dev, rtol=0, atol=1e-10)


def test_fan_out_add_equals_chain_with_summed_weight():
    g = torch.Generator().manual_seed(4)
    W1 = torch.randn(20, 8, generator=g, dtype=torch.float64)
    b1 = torch.randn(20, generator=g, dtype=torch.float64) * 0.5
    W2 = torch.randn(16, 20, generator=g, dtype=torch.float64)
    b2 = torch.randn(16, generator=g, dtype=torch.float64)
    W3 = torch.randn(16, 20, generator=g, dtype=torch.float64)
    b3 = torch.randn(16, generator=g, dtype=torch.float64)
    W4 = torch.randn(5, 16, generator=g, dtype=torch.float64)
    b4 = torch.randn(5, generator=g, dtype=torch.float64)
    dag = _module([
        TaskOp("linear", "lin1", ["input", "W1", "b1"], ["h1"]),
        TaskOp("relu", "relu1", ["h1"], ["r1"]),
        TaskOp("linear", "lin2", ["r1", "W2", "b2"], ["h2"]),
        TaskOp("linear", "lin3", ["r1", "W3", "b3"], ["h3"]),
        TaskOp("add", "add0", ["h2", "h3"], ["s"]),
        TaskOp("relu", "relu2", ["s"], ["r2"]),
        TaskOp("linear", "lin4", ["r2", "W4", "b4"], ["out"]),
    ], {"W1": W1, "b1": b1, "W2": W2, "b2": b2, "W3": W3, "b3": b3, "W4": W4, "b4": b4})
    chain = _module([
        TaskOp("linear", "lin1", ["input", "W1", "b1"], ["h1"]),
        TaskOp("relu", "relu1", ["h1"], ["r1"]),
        TaskOp("linear", "lin23", ["r1", "W23", "b23"], ["s"]),
        TaskOp("relu", "relu2", ["s"], ["r2"]),
        TaskOp("linear", "lin4", ["r2", "W4", "b4"], ["out"]),
    ], {"W1": W1, "b1": b1, "W23": W2 + W3, "b23": b2 + b3, "W4": W4, "b4": b4})
    x = torch.rand(3, 8, generator=g, dtype=torch.float64)
    spec = InputSpec.linf(value_name="input", center=x, eps=0.2)
    C = torch.randn(3, 4, 5, generator=g, dtype=torch.float64)
    env_d, pre_d = cr.forward_ibp_trace(dag, spec)
    env_c, pre_c = cr.forward_ibp_trace(chain, spec)
    assert _ambiguous_count(pre_c) > 0
    # the intermediate box of s differs (IBP of a sum is looser than IBP of the summed
    # layer), so both backward passes take the chain's pre-activation boxes
    d = cr.crown_backward_from_trace(dag, spec, interval_env=env_d, relu_pre=pre_c, linear_spec_C=C)
    c = cr.crown_backward_from_trace(chain, spec, interval_env=env_c, relu_pre=pre_c, linear_spec_C=C)
    torch.testing.assert_close(d.lower, c.lower, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(d.upper, c.upper, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("conv", [False, True])
def test_concat_equals_chain_with_stacked_weight(conv):
    g = torch.Generator().manual_seed(6)
    if conv:
        W1 = torch.randn(3, 2, 3, 3, generator=g, dtype=torch.float64)
        W2 = torch.randn(4, 2, 3, 3, generator=g, dtype=torch.float64)
        n1, n2, flat = 3, 4, 7 * 36
        x = torch.rand(2, 2, 6, 6, generator=g, dtype=torch.float64)
        attrs = {"stride": 1, "padding": 1}
        kind = "conv2d"
    else:
        W1 = torch.randn(9, 6, generator=g, dtype=torch.float64)
        W2 = torch.randn(5, 6, generator=g, dtype=torch.float64)
        n1, n2, flat = 9, 5, 14
        x = torch.rand(2, 6, generator=g, dtype=torch.float64)
        attrs = {}
        kind = "linear"
    b1 = torch.randn(n1, generator=g, dtype=torch.float64)
    b2 = torch.randn(n2, generator=g, dtype=torch.float64)
    W3 = torch.randn(4, flat, generator=g, dtype=torch.float64)
    b3 = torch.randn(4, generator=g, dtype=torch.float64)
    tail = ([TaskOp("flatten", "flat", ["r"], ["f"], {"start_dim": 1, "end_dim": -1})] if conv else [])
    head_in = "f" if conv else "r"
    dag = _module([
        TaskOp(kind, "a1", ["input", "W1", "b1"], ["h1"], dict(attrs)),
        TaskOp(kind, "a2", ["input", "W2", "b2"], ["h2"], dict(attrs)),
        TaskOp("concat", "cat", ["h1", "h2"], ["h"], {"axis": 1}),
        TaskOp("relu", "relu", ["h"], ["r"]),
        *tail,
        TaskOp("linear", "head", [head_in, "W3", "b3"], ["out"]),
    ], {"W1": W1, "b1": b1, "W2": W2, "b2": b2, "W3": W3, "b3": b3})
    chain = _module([
        TaskOp(kind, "a12", ["input", "W12", "b12"], ["h"], dict(attrs)),
        TaskOp("relu", "relu", ["h"], ["r"]),
        *tail,
        TaskOp("linear", "head", [head_in, "W3", "b3"], ["out"]),
    ], {"W12": torch.cat([W1, W2]), "b12": torch.cat([b1, b2]), "W3": W3, "b3": b3})
    spec = InputSpec.linf(value_name="input", center=x, eps=0.1)
    env_d, pre_d = cr.forward_ibp_trace(dag, spec)
    env_c, pre_c = cr.forward_ibp_trace(chain, spec)
    assert _ambiguous_count(pre_c) > 0
    for name in pre_c:       # IBP rows are independent: the concatenated box is the stacked layer's box
        torch.testing.assert_close(pre_d[name].lower, pre_c[name].lower, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(pre_d[name].upper, pre_c[name].upper, rtol=1e-12, atol=1e-12)
    d = cr.crown_backward_from_trace(dag, spec, interval_env=env_d, relu_pre=pre_d)
    c = cr.crown_backward_from_trace(chain, spec, interval_env=env_c, relu_pre=pre_c)
    torch.testing.assert_close(d.lower, c.lower, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(d.upper, c.upper, rtol=1e-12, atol=1e-12)


def test_dag_rejects_broadcast_add_and_bad_concat_axis():
    """tests/test_phase7a_pr8_general_dag_runtime.py:341-363."""
    g = torch.Generator().manual_seed(8)
    W1 = torch.randn(4, 3, generator=g, dtype=torch.float64)
    x = torch.rand(2, 3, generator=g, dtype=torch.float64)
    spec = InputSpec.linf(value_name="input", center=x, eps=0.1)
    bcast = _module([
        TaskOp("linear", "lin1", ["input", "W1"], ["h1"]),
        TaskOp("add", "add0", ["h1", "c"], ["s"]),
        TaskOp("linear", "lin2", ["s", "W2"], ["out"]),
    ], {"W1": W1, "c": torch.ones(4, dtype=torch.float64), "W2": torch.randn(2, 4, generator=g,
                                                                              dtype=torch.float64)})
    with pytest.raises(NotImplementedError, match="same-shape"):
        cr.forward_ibp_trace(bcast, spec)
    axis0 = _module([
        TaskOp("linear", "lin1", ["input", "W1"], ["h1"]),
        TaskOp("linear", "lin2", ["input", "W1"], ["h2"]),
        TaskOp("concat", "cat", ["h1", "h2"], ["h"], {"axis": 0}),
        TaskOp("linear", "lin3", ["h", "W3"], ["out"]),
    ], {"W1": W1, "W3": torch.randn(2, 8, generator=g, dtype=torch.float64)})
    with pytest.raises(NotImplementedError, match="axis"):
        cr.forward_ibp_trace(axis0, spec)
