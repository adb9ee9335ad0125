"""The PyTorch frontend, planner v0 and the VNNLIB parser (CPU).

* ``import_torch`` + ``plan_interval_ibp_v0`` of nn.Module versions of C1, C3 and
  the reference's DAG frontend nets (residual add, concat) and a layout-only
  permute net: every field the backend reads (ops, attrs, task values and
  buffers, storage plan, parameter shapes) equals the reference planner's output
  (fixture ``frontend_planned``, written by tests/golden/make_golden.py);
* the planned C1 and C3 modules give the oracle bounds of the hand-built
  workloads bit for bit;
* ``parse_vnnlib_box_query``: the reference's known answers
  (tests/test_vnnlib_query_ir.py of the reference), its rejections, and the query
  IR dict and stable hash of three sources (fixture ``vnnlib_queries``)."""

import hashlib
import json

import pytest
import torch

from boundflow_amd import frontend as fe
from boundflow_amd import vnnlib as vn
from boundflow_amd import workloads as wl
from boundflow_amd.spec import InputSpec
from oracle import crown_ref as cr
from tests.frontend_models import (VNNLIB_SOURCES, frontend_nets, planned_module_json, sequential_from_chain,
                                   vnnlib_c1_property)
from tests.golden_util import load


@pytest.mark.parametrize("name", ["c1_mlp", "c3_cnn", "residual_add", "concat", "permute"])
def test_planned_module_matches_reference_planner(name):
    g = load("frontend_planned")
    net, x = frontend_nets()[name]
    tm = fe.plan_interval_ibp_v0(fe.import_torch(net, (x,)))
    got = json.loads(planned_module_json(tm))
    ref = json.loads(str(g[name]))
    assert got["task"] == ref["task"]
    assert got["ops"] == ref["ops"]
    assert got["buffers"] == ref["buffers"]
    assert got["value_to_buffer"] == ref["value_to_buffer"]
    assert got["param_shapes"] == ref["param_shapes"]


def test_fx_mode_and_value_kinds():
    net, x = frontend_nets()["c1_mlp"]
    prog = fe.import_torch(net, (x,))
    assert prog.graph.inputs == ["input"] and len(prog.graph.outputs) == 1
    assert prog.graph.values["input"].kind == fe.ValueKind.INPUT
    assert all(prog.graph.values[k].kind == fe.ValueKind.PARAM for k in prog.params)
    # fx mode: parameters are get_attr constants; leaf modules (call_module) are refused, as in the reference
    with pytest.raises(NotImplementedError, match="call_module"):
        fe.import_torch(net, (x,), export_mode="fx")

    class Functional(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.w = torch.nn.Parameter(torch.randn(3, 4))

        def forward(self, v):
            return torch.relu(v @ self.w.t()).flatten(1)

    fx = fe.import_torch(Functional(), (torch.randn(2, 4),), export_mode="fx")
    kinds = {v.kind for v in fx.graph.values.values()}
    assert fe.ValueKind.CONST in kinds and fx.graph.inputs == ["v"]
    with pytest.raises(ValueError, match="unsupported export_mode"):
        fe.import_torch(net, (x,), export_mode="onnx")


@pytest.mark.parametrize("name", ["C1", "C3"])
def test_planned_workload_bounds_are_bit_identical(name):
    w = wl.subset(wl.make(name), 6)
    net = sequential_from_chain(w.module)
    example = w.spec.perturbation.lower if name == "C1" else w.spec.center
    tm = fe.plan_interval_ibp_v0(fe.import_torch(net, (example,)))
    spec = InputSpec(value_name="input", center=w.spec.center, perturbation=w.spec.perturbation)
    a = cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C)
    b = cr.run_crown_ibp(tm, spec, linear_spec_C=w.C)
    assert torch.equal(a.lower, b.lower) and torch.equal(a.upper, b.upper)


SOURCE = VNNLIB_SOURCES["reference_example"]


def test_vnnlib_known_answers():
    q = vn.parse_vnnlib_box_query(SOURCE, query_id="classification:0")
    assert q.source_sha256 == hashlib.sha256(SOURCE.encode()).hexdigest()
    assert q.input_names == ("X_0", "X_1") and q.output_names == ("Y_0", "Y_1", "Y_2")
    assert q.input_lower == (-1.0, 0.25) and q.input_upper == (2.0, 3.5)
    assert q.unsafe_clauses[0].coefficients == (-1.0, 0.0, 1.0)
    assert q.unsafe_clauses[1].coefficients == (0.0, 1.0, -1.0)
    assert tuple(c.threshold for c in q.unsafe_clauses) == (0.0, 0.0)
    t = vn.materialize_vnnlib_box_query(q, input_shape=(2,), dtype=torch.float64)
    assert t.input_lower.shape == (1, 2) and t.linear_spec_c.shape == (1, 2, 3) and t.thresholds.shape == (2,)
    assert torch.equal(t.linear_spec_c, torch.tensor([[[-1.0, 0.0, 1.0], [0.0, 1.0, -1.0]]], dtype=torch.float64))
    q2 = vn.parse_vnnlib_box_query(SOURCE.replace("(and (>= Y_0 Y_2))", "(and (>= (+ Y_0 1.5) (* 2.0 Y_2)))"),
                                   query_id="linear:0")
    assert q2.unsafe_clauses[0].coefficients == (-1.0, 0.0, 2.0) and q2.unsafe_clauses[0].threshold == 1.5


@pytest.mark.parametrize("source, message", [
    (SOURCE.replace("(assert (<= X_0 2.0))", ""), "incomplete"),
    (SOURCE.replace("(assert (<= X_0 2.0))", "(assert (<= X_0 2.0))\n(assert (<= X_0 1.0))"), "duplicates"),
    (SOURCE.replace("X_1", "X_2"), "Query IR is invalid"),
    (SOURCE.replace("(and (>= Y_0 Y_2))", "(and (>= Y_0 Y_2) (>= Y_1 Y_2))"), "one inequality"),
    (SOURCE.replace("(>= Y_0 Y_2)", "(= Y_0 Y_2)"), "unsupported"),
    (SOURCE + ")", "unmatched closing"),
    ("(declare-const X_0 Real", "unmatched opening"),
    (SOURCE.replace("(<= Y_1 Y_2)", "(<= Y_1 X_0)"), "cannot mix"),
])
def test_vnnlib_rejections(source, message):
    with pytest.raises(ValueError, match=message):
        vn.parse_vnnlib_box_query(source, query_id="invalid")


def test_vnnlib_digest_and_shape_checks():
    with pytest.raises(ValueError, match="digest differs"):
        vn.parse_vnnlib_box_query(SOURCE, query_id="classification:0", expected_source_sha256="0" * 64)
    q = vn.parse_vnnlib_box_query(SOURCE, query_id="classification:0")
    with pytest.raises(ValueError, match="shape/dtype differs"):
        vn.materialize_vnnlib_box_query(q, input_shape=(3,))


@pytest.mark.parametrize("name", ["reference_example", "linear_terms", "c1_property0"])
def test_vnnlib_query_matches_reference_parser(name):
    g = json.loads(str(load("vnnlib_queries")[name]))
    text = vnnlib_c1_property(0) if name == "c1_property0" else VNNLIB_SOURCES[name]
    q = vn.parse_vnnlib_box_query(text, query_id=f"{name}:0")
    assert q.to_dict() == g["dict"]
    assert q.stable_hash() == g["stable_hash"]


def test_vnnlib_property_runs_through_the_oracle():
    """The C1 property: its box and clause matrix give the same bounds as the
    hand-built C1 query on that input (the clauses are the margin rows of C1's spec
    with the opposite sign: unsafe when Y_j - Y_y >= 0)."""
    w = wl.subset(wl.make_c1(), 1)
    q = vn.parse_vnnlib_box_query(vnnlib_c1_property(0), query_id="c1:0")
    t = vn.materialize_vnnlib_box_query(q, input_shape=(784,))
    spec = InputSpec.box(value_name="input", lower=t.input_lower, upper=t.input_upper)
    b = cr.run_crown_ibp(w.module, spec, linear_spec_C=t.linear_spec_c)
    ref = cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C)
    assert torch.equal(b.lower, ref.lower) and torch.equal(b.upper, ref.upper)
    assert vn.query_verified(b.lower, t.thresholds) == bool((ref.lower > 0).all())
