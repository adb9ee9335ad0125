"""get_crown_ibp_mlp_stats (crown_ibp.py:2279-2350): which modules run_crown_ibp_mlp takes,
with the reason for those it does not (as tests/test_phase6b_crown_ibp_mlp.py:269 and
tests/test_phase7a_pr3_crown_ibp_cnn.py:175-195 use it)."""

import torch

from boundflow_amd import workloads as wl
from boundflow_amd.crown import get_crown_ibp_mlp_stats
from boundflow_amd.ir import BFTaskModule, BoundTask, TaskKind, TaskOp


def _module(ops, params):
    task = BoundTask(task_id="t0", kind=TaskKind.INTERVAL_IBP, ops=ops, input_values=["input"],
                     output_values=[ops[-1].outputs[0]])
    return BFTaskModule(tasks=[task], entry_task_id="t0", bindings={"params": params})


def test_supported_chains_and_dags():
    for w in (wl.make_c1(batch=2), wl.make_c3(batch=2), wl.make_dag("residual_mlp", batch=2),
              wl.make_dag("channel_concat_cnn", batch=2)):
        st = get_crown_ibp_mlp_stats(w.module)
        assert st.supported, (w.name, st.reason)
        assert st.ops_seen == tuple(op.op_type for op in w.module.get_entry_task().ops)


def test_unsupported_modules_give_a_reason():
    W, b = torch.randn(3, 4), torch.randn(3)
    bad_op = _module([TaskOp("linear", "l1", ["input", "W", "b"], ["h"]), TaskOp("sigmoid", "s", ["h"], ["o"])],
                     {"W": W, "b": b})
    st = get_crown_ibp_mlp_stats(bad_op)
    assert not st.supported and "sigmoid" in st.reason
    bad_flat = _module([TaskOp("flatten", "f", ["input"], ["x"], attrs={"start_dim": 0}),
                        TaskOp("linear", "l1", ["x", "W", "b"], ["o"])], {"W": W, "b": b})
    st = get_crown_ibp_mlp_stats(bad_flat)
    assert not st.supported and "flatten" in st.reason
    Wc = torch.randn(2, 1, 3, 3)
    grouped = _module([TaskOp("conv2d", "c", ["input", "Wc"], ["o"], attrs={"dilation": 2})], {"Wc": Wc})
    st = get_crown_ibp_mlp_stats(grouped)
    assert not st.supported and "dilation" in st.reason
