"""The native ReLU-split queue on the device (bab.run_native_relu_split_bab)
against whole runs of the reference's run_native_relu_split_bab (fixtures
native_*, written by tests/golden/make_golden.py): identical node ids, lineage,
prune / expand / terminal decisions and reasons, branch choices, final frontier,
status, largest queue and number of evaluated batches; node bounds within the
contract (1e-5 relative, 1e-6 absolute)."""

import json

import pytest

from boundflow_amd import bab as hbab
from boundflow_amd import workloads as wl
from boundflow_amd.ir import BFTaskModule
from boundflow_amd.spec import InputSpec
from tests.golden_util import load
from tests.gpu_util import announce, device
from tests.test_oracle_bab import NATIVE, compare_native, native_problem

pytestmark = pytest.mark.gpu


def _as_dict(trace):
    def br(b):
        return None if b is None else [b.relu_input, b.neuron_index, b.lower, b.upper, b.width]
    return {"status": trace.status, "frontier": list(trace.final_frontier_node_ids),
            "max_queue_size": trace.max_queue_size, "stacks": trace.native_stack_count,
            "evaluations": [{"node_id": e.node_id, "parent": e.parent_node_id, "depth": e.depth, "lower": e.lower,
                             "upper": e.upper, "priority": e.priority, "branch": br(e.branch_candidate)}
                            for e in trace.evaluations],
            "decisions": [{"node_id": d.node_id, "kind": d.kind, "reason": d.reason,
                           "children": list(d.child_node_ids), "branch": br(d.branch_candidate)}
                          for d in trace.decisions]}


@pytest.mark.parametrize("tag", list(NATIVE))
def test_native_queue_matches_reference(tag):
    dev = device()
    announce(f"native ReLU-split queue {tag}")
    kind, cfg = NATIVE[tag]
    module, spec, C = native_problem(kind)
    md = BFTaskModule(tasks=module.tasks, entry_task_id=module.entry_task_id,
                      bindings={"params": {k: v.to(dev) for k, v in module.params.items()}})
    sd = InputSpec.box(value_name=spec.value_name, lower=spec.perturbation.lower.to(dev),
                       upper=spec.perturbation.upper.to(dev))
    trace = hbab.run_native_relu_split_bab(md, sd, linear_spec_C=C.to(dev), run_id=tag,
                                           config=hbab.NativeReluSplitBabConfig(**cfg))
    got = _as_dict(trace)
    ref = json.loads(str(load(tag)["trace"]))
    announce(f"  {got['status']}: {len(got['evaluations'])} evaluations, {len(got['decisions'])} decisions, "
             f"{got['stacks']} batches")
    compare_native(got, ref)
    assert got["stacks"] == ref["stacks"]
