"""Host-side logic of the drop-in executors (no device needed): fused-region
planning and validation (runtime/fused_crown.py:178-276), runtime selection
(:826-847), TaskGraph ordering and validation (ir/task_graph.py:37-168), and the
errors the IBP task executor raises before it launches anything."""

import dataclasses

import pytest
import torch

from boundflow_amd import fused_crown as fc
from boundflow_amd import task_executor as te
from boundflow_amd import workloads as wl
from boundflow_amd.ir import TaskBufferDep, TaskDepEdge, TaskGraph, TaskOp


def test_plan_matches_every_affine_relu_pair():
    ops = wl.make_c1().module.get_entry_task().ops   # linear0 relu0 linear1 relu1 linear2
    steps = fc.plan_fused_crown_regions(ops)
    assert [(s.kind, s.affine_op_index, s.relu_op_index) for s in steps] == [
        ("fused_relu_linear", 0, 1), ("fused_relu_linear", 2, 3)]
    assert all(s.backend == "hip_fused" for s in steps)
    assert steps[0].consumed_outputs == ("r0", "h0")
    assert fc.validate_fused_crown_execution_steps(ops, steps) == steps


def test_plan_conv_regions_and_skips_shared_affine_output():
    ops = list(wl.make_c3().module.get_entry_task().ops)
    steps = fc.plan_fused_crown_regions(ops)
    assert [s.kind for s in steps] == ["fused_relu_conv2d", "fused_relu_conv2d", "fused_relu_linear"]
    # a second consumer of the conv output makes the region unfusable
    ops.append(TaskOp("relu", "extra", ["h0"], ["h0b"]))
    kinds = [(s.affine_op_index, s.relu_op_index) for s in fc.plan_fused_crown_regions(ops)]
    assert (0, 1) not in kinds


def test_validate_drops_stale_and_malformed_steps():
    ops = wl.make_c1().module.get_entry_task().ops
    steps = fc.plan_fused_crown_regions(ops)
    stale = dataclasses.replace(steps[0], graph_fingerprint="0" * 64)
    wrong_kind = dataclasses.replace(steps[1], kind="fused_relu_conv2d")
    dup = steps[0]
    assert fc.validate_fused_crown_execution_steps(ops, [stale, wrong_kind]) == ()
    assert fc.validate_fused_crown_execution_steps(ops, [steps[0], dup]) == (steps[0],)
    with pytest.raises(ValueError):
        fc.plan_fused_crown_regions(ops, backend="cuda_magic")


def test_runtime_selection():
    ops = wl.make_c1().module.get_entry_task().ops
    sel = fc.build_fused_crown_runtime_selection(ops, backend="hip_fused")
    assert isinstance(sel.executor, fc.HipFusedCrownExecutor) and len(sel.steps) == 2
    eager = fc.build_fused_crown_runtime_selection(ops, backend="pytorch_eager")
    assert eager.executor is None and eager.steps == ()
    with pytest.raises(ValueError):
        fc.build_fused_crown_runtime_selection(ops, backend="tvm_fused_tir")


def test_descriptor_support():
    ex = fc.HipFusedCrownExecutor()
    ctx = fc.FusedCrownExecutionContext()
    w = torch.zeros(4, 3, 4, 4)
    d = fc.FusedReluAffineDescriptor(kind="conv2d", coefficient_shape=(2, 9, 64), weight=w, bias=None,
                                     input_shape=(3, 8, 8), output_shape=(4, 4, 4),
                                     attrs={"stride": 2, "padding": 1}, device=torch.device("cuda", 0),
                                     dtype=torch.float32)
    assert ex.supports_descriptor(d, ctx)
    assert not ex.supports_descriptor(d, fc.FusedCrownExecutionContext(requires_grad=True))
    assert not ex.supports_descriptor(dataclasses.replace(d, attrs={"groups": 2}), ctx)
    assert not ex.supports_descriptor(dataclasses.replace(d, dtype=torch.float64), ctx)
    assert not ex.supports_descriptor(dataclasses.replace(d, device=torch.device("cpu")), ctx)


def test_task_graph_order_and_errors():
    w = wl.make_ibp_dag()
    m = wl.split_ibp_dag(w)
    tasks = {t.task_id: t for t in m.tasks}
    assert m.task_graph.topo_sort(tasks_by_id=tasks, entry_task_id="t0") == ["t0", "t1", "t2"]
    cyc = TaskGraph(task_ids=["t0", "t1"], edges=[TaskDepEdge("t0", "t1", []), TaskDepEdge("t1", "t0", [])])
    with pytest.raises(ValueError, match="cycle"):
        cyc.topo_sort(tasks_by_id=tasks, entry_task_id="t0")
    bad = TaskGraph(task_ids=["t0", "t1", "t2"], edges=[
        TaskDepEdge("t0", "t1", [TaskBufferDep("r0", "buf_h0", "r0", "buf_r0")])])
    with pytest.raises(ValueError):
        bad.validate(tasks_by_id=tasks, entry_task_id="t0", storage_plan=m.storage_plan)
    chain = TaskGraph.chain("a", "b", "c")
    assert [(e.src_task_id, e.dst_task_id) for e in chain.edges] == [("a", "b"), ("b", "c")]


def test_task_executor_errors_before_launch():
    w = wl.make_ibp_dag()
    m = wl.split_ibp_dag(w)
    t1 = m.get_task("t1")
    plan = m.storage_plan
    env = {}
    with pytest.raises(KeyError, match="missing value"):
        te.HipTaskExecutor().run_ibp_task(t1, env=env, params=m.params, storage_plan=plan)
    broken = dataclasses.replace(plan, value_to_buffer={k: v for k, v in plan.value_to_buffer.items() if k != "r0"})
    with pytest.raises(KeyError, match="not found in storage_plan"):
        te.HipTaskExecutor().run_ibp_task(t1, env=env, params=m.params, storage_plan=broken)
    with pytest.raises(ValueError, match="not in task.input_values"):
        from boundflow_amd.spec import InputSpec
        te.HipTaskExecutor().run_ibp(w.module, InputSpec.linf(value_name="x", center=w.spec.center, eps=0.1))
    from boundflow_amd.spec import InputSpec, LpBallPerturbation
    l2 = InputSpec(value_name="input", center=w.spec.center, perturbation=LpBallPerturbation(p=2, eps=0.1))
    with pytest.raises(NotImplementedError):
        te.run_ibp_scheduled(m, l2)
