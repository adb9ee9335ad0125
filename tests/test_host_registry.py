"""The typed-registry entry of the HIP backend (boundflow_amd.fused_crown.
HipTaskBackendRegistry), checked with stand-ins for the reference's Task IR unit,
dispatch key, plan template and Bound IR session: the dispatch contract of
TVMTaskBackendRegistry.dispatch (boundflow/runtime/task_backend_dispatch.py:435-495).
No device call is made."""

from dataclasses import dataclass, field
from types import SimpleNamespace as NS

import pytest

from boundflow_amd.fused_crown import HipFusedCrownExecutor, HipTaskBackendRegistry


@dataclass
class _Session:
    calls: list = field(default_factory=list)

    def execute_fused_relu_affine_task(self, op_ids, *, output_value_ids, executor):
        self.calls.append((op_ids, output_value_ids, executor))
        return ("result", op_ids)


def _op(op_id, kind):
    return NS(op_id=op_id, kind=NS(value=kind))


def _case(kinds=("relu_relaxation", "linear_backward"), backend="hip_fused", digest="k1", task_id="t0"):
    task = NS(task_id=task_id, op_refs=[_op(f"op{i}", k) for i, k in enumerate(kinds)], output_value_ids=("v",))
    template = NS(backend_candidates=[NS(candidate_id="c0", backend=NS(value=backend), capability_id="cap")])
    key = NS(backend_candidate_id="c0", stable_hash=lambda: digest)
    return task, key, template


def test_dispatch_runs_the_fused_region_through_the_hip_executor():
    reg, sess = HipTaskBackendRegistry(), _Session()
    task, key, template = _case()
    out = reg.dispatch(task, key, session=sess, template=template)
    assert out == ("result", ("op0", "op1"))
    (op_ids, outs, executor), = sess.calls
    assert op_ids == ("op0", "op1") and outs == ("v",) and isinstance(executor, HipFusedCrownExecutor)
    reg.dispatch(task, key, session=sess, template=template)
    assert (reg.cache_misses, reg.cache_hits) == (1, 1)
    task_c, key_c, template_c = _case(kinds=("relu_relaxation", "conv2d_backward"), digest="k2")
    reg.dispatch(task_c, key_c, session=sess, template=template_c)
    assert reg.cache_misses == 2


@pytest.mark.parametrize("kinds,backend,msg", [
    (("relu_relaxation", "linear_backward"), "tvm_fused_tir", "rejects backend"),
    (("linear_backward",), "hip_fused", "fused ReLU->Affine"),
    (("relu_relaxation", "add_backward"), "hip_fused", "fused ReLU->Affine"),
])
def test_dispatch_rejects_other_backends_and_tasks(kinds, backend, msg):
    task, key, template = _case(kinds=kinds, backend=backend)
    with pytest.raises(ValueError, match=msg):
        HipTaskBackendRegistry().dispatch(task, key, session=_Session(), template=template)


def test_unknown_candidate_and_key_collision():
    reg = HipTaskBackendRegistry()
    task, key, template = _case()
    with pytest.raises(ValueError, match="unknown backend"):
        reg.dispatch(task, NS(backend_candidate_id="zz", stable_hash=lambda: "k"), session=_Session(),
                     template=template)
    reg.dispatch(task, key, session=_Session(), template=template)
    other, _k, _t = _case(task_id="t9")
    with pytest.raises(ValueError, match="collision"):
        reg.dispatch(other, key, session=_Session(), template=template)
