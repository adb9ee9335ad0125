"""Pin the branch-and-bound oracle (oracle/bab_ref.py).

* against whole searches of the reference's solve_bab_mlp (tests/golden,
  written by tests/golden/make_golden.py): statuses, node counts, rounds, queue
  size, fill rate and best bounds;
* by what a verdict means: a "proven" example has no sampled point of its input
  ball with a negative margin; an "unsafe" one has a point that violates
  (found by projected gradient descent on the margin, or by sampling).
"""

import numpy as np
import pytest
import torch

from boundflow_amd import workloads as wl
from oracle import bab_ref
from tests.golden_util import (ALPHA_CROWN_OBJECTIVE_CASES, BAB_SOLVE_CASES, OBJECTIVE_CASES, load, objective_workload,
                               workload_checksum)

CASES = BAB_SOLVE_CASES
DEFAULTS = dict(use_branch_hint=True, alpha_lr=0.2, alpha_init=0.5, beta_init=0.0, threshold=0.0, tol=1e-6)
CODE = {"proven": 0, "unsafe": 1, "unknown": 2}


def config(tag):
    toy, kw = CASES[tag]
    return toy, {**DEFAULTS, **kw}


@pytest.mark.parametrize("tag", list(CASES))
def test_bab_search_matches_reference(tag):
    g = load(tag)
    toy, cfg = config(tag)
    w = wl.make_bab_case(**toy)
    assert workload_checksum(w) == str(g["checksum"])
    r = bab_ref.solve_bab_mlp(w.module, w.spec, linear_spec_C=w.C, config=cfg)
    assert CODE[r["status"]] == int(g["status"])
    assert [CODE[s] for s in r["per_status"]] == g["per_status"].tolist()
    for k in ("nodes_visited", "nodes_evaluated", "nodes_expanded", "max_queue", "batch_rounds"):
        assert r[k] == int(g[k]), k
    assert r["per_visited"] == g["per_visited"].tolist()
    assert r["per_evaluated"] == g["per_evaluated"].tolist()
    assert r["per_expanded"] == g["per_expanded"].tolist()
    assert abs(r["avg_batch_fill_rate"] - float(g["avg_batch_fill_rate"])) < 1e-12
    np.testing.assert_allclose(r["per_best_lower"], g["per_best_lower"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(r["per_best_upper"], g["per_best_upper"], rtol=1e-5, atol=1e-6)


def _margins(w, x):
    p = {k: v.double() for k, v in w.module.params.items()}
    h = x.double()
    ops = [op for op in w.module.get_entry_task().ops]
    for op in ops:
        if op.op_type == "linear":
            h = h @ p[op.inputs[1]].t() + p[op.inputs[2]]
        elif op.op_type == "relu":
            h = h.clamp_min(0)
    return torch.einsum("bso,bo->bs", w.C.double(), h)


@pytest.mark.parametrize("tag", ["bab_solve_ab_e003", "bab_solve_ab_e005"])
def test_bab_verdicts_are_sound(tag):
    toy, cfg = config(tag)
    eps = toy["eps"]
    w = wl.make_bab_case(**toy)
    r = bab_ref.solve_bab_mlp(w.module, w.spec, linear_spec_C=w.C, config=cfg)
    x0 = w.spec.center.double()
    g = torch.Generator().manual_seed(9)
    for e, st in enumerate(r["per_status"]):
        if st == "proven":
            pts = x0[e] + eps * (2 * torch.rand(4000, x0.shape[1], generator=g, dtype=torch.float64) - 1)
            corners = x0[e] + eps * torch.sign(torch.randn(4000, x0.shape[1], generator=g, dtype=torch.float64))
            xs = torch.cat([pts, corners])
            C = w.C[e:e + 1].double().expand(xs.shape[0], -1, -1)
            ww = type(w)(w.name, w.module, w.spec, C, w.labels)
            assert float(_margins(ww, xs).min()) >= -1e-9, f"example {e} proven but a sampled point violates"
        if st == "unsafe":
            # projected gradient descent on the smallest margin from many starts
            xs = (x0[e] + eps * (2 * torch.rand(256, x0.shape[1], generator=g, dtype=torch.float64) - 1))
            xs.requires_grad_(True)
            C = w.C[e:e + 1].double().expand(xs.shape[0], -1, -1)
            ww = type(w)(w.name, w.module, w.spec, C, w.labels)
            for _ in range(200):
                m = _margins(ww, xs).min(dim=1).values
                (gx,) = torch.autograd.grad(m.sum(), xs)
                with torch.no_grad():
                    xs -= eps * 0.05 * gx.sign()
                    xs.copy_(torch.maximum(torch.minimum(xs, x0[e] + eps), x0[e] - eps))
            assert float(_margins(ww, xs.detach()).min()) < 0, f"example {e} unsafe but no violating point found"


NATIVE = {
    "native_toy_b4": ("toy", dict(max_nodes=15, max_depth=3, expansion_batch_size=2, max_eval_batch_size=4,
                                  threshold=1e6)),
    "native_toy_budget": ("toy", dict(max_nodes=7, max_depth=3, expansion_batch_size=2, max_eval_batch_size=4,
                                      threshold=1e6)),
    "native_mlp": ("mlp", dict(max_nodes=41, max_depth=6, expansion_batch_size=3, max_eval_batch_size=8,
                               threshold=0.0)),
}


def native_problem(kind):
    from tests.frontend_models import native_bab_toy, native_toy
    return native_toy() if kind == "toy" else native_bab_toy()


def compare_native(got: dict, ref: dict, bound_tol=(1e-5, 1e-6)):
    """Identical queue: statuses, node ids, lineage, decisions, branch choices, frontier; bounds within tolerance."""
    rtol, atol = bound_tol
    assert got["status"] == ref["status"]
    assert got["frontier"] == ref["frontier"]
    assert got["max_queue_size"] == ref["max_queue_size"]
    assert len(got["evaluations"]) == len(ref["evaluations"])
    for g, r in zip(got["evaluations"], ref["evaluations"]):
        assert (g["node_id"], g["parent"], g["depth"]) == (r["node_id"], r["parent"], r["depth"])
        for k in ("lower", "upper"):
            assert abs(g[k] - r[k]) <= atol + rtol * abs(r[k]), (g["node_id"], k, g[k], r[k])
        gb, rb = g["branch"], r["branch"]
        assert (gb is None) == (rb is None) and (gb is None or list(gb[:2]) == list(rb[:2])), g["node_id"]
    assert len(got["decisions"]) == len(ref["decisions"])
    for g, r in zip(got["decisions"], ref["decisions"]):
        assert (g["node_id"], g["kind"], g["reason"]) == (r["node_id"], r["kind"], r["reason"])
        assert list(g.get("children", [])) == list(r["children"])
        assert (g.get("branch") is None) == (r["branch"] is None)
        if r["branch"] is not None:
            assert list(g["branch"][:2]) == list(r["branch"][:2])


@pytest.mark.parametrize("tag", list(NATIVE))
def test_native_queue_matches_reference(tag):
    import json
    kind, cfg = NATIVE[tag]
    module, spec, C = native_problem(kind)
    ref = json.loads(str(load(tag)["trace"]))
    got = bab_ref.run_native_relu_split_bab(module, spec, linear_spec_C=C, run_id=tag, **cfg)
    compare_native(got, ref)
    assert got["stacks"] == ref["stacks"]


@pytest.mark.parametrize("case", list(OBJECTIVE_CASES))
def test_objectives_match_reference(case):
    """The oracle's objectives and spec reductions (alpha_beta_crown.py:756-815) against
    the reference's run_alpha_beta_crown_mlp on the same problem (fixture objectives_mlp)."""
    from oracle import alpha_beta_ref as ab
    g = load("objectives_mlp")
    w, splits = objective_workload()
    assert workload_checksum(w) == str(g["checksum"])
    for n, v in splits.items():
        assert torch.equal(v, torch.from_numpy(g[f"split_{n}"]))
    b, _a, _bt, _ch = ab.run_alpha_beta_crown(w.module, w.spec, linear_spec_C=w.C, relu_split_state=splits, steps=8,
                                              lr=0.1, **OBJECTIVE_CASES[case])
    np.testing.assert_allclose(b.lower.numpy(), g[f"{case}_lower"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(b.upper.numpy(), g[f"{case}_upper"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("case", list(ALPHA_CROWN_OBJECTIVE_CASES))
def test_alpha_crown_objectives_match_reference(case):
    """The oracle's shared-alpha objectives (alpha_crown.py:62-135, whole-[B, S]
    "mean") against the reference's run_alpha_crown_mlp (fixture
    alpha_crown_objectives): best bounds and best alpha after 8 Adam steps."""
    from oracle import alpha_beta_ref as ab
    g = load("alpha_crown_objectives")
    w, splits = objective_workload()
    assert workload_checksum(w) == str(g["checksum"])
    b, alpha = ab.run_alpha_crown(w.module, w.spec, linear_spec_C=w.C, relu_split_state=splits, steps=8, lr=0.1,
                                  **ALPHA_CROWN_OBJECTIVE_CASES[case])
    np.testing.assert_allclose(b.lower.detach().numpy(), g[f"{case}_lower"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(b.upper.detach().numpy(), g[f"{case}_upper"], rtol=1e-5, atol=1e-6)
    for n, a in alpha.items():
        np.testing.assert_allclose(a.numpy(), g[f"{case}_alpha_{n}"], rtol=1e-5, atol=1e-6)


def test_alpha_oracle_refuses_conv_graphs():
    """bab.py:656-659: the alpha-only search does not take conv graphs."""
    w = wl.make_bab_cnn_toy(seed=2, eps=0.01, channels=2, hidden=16, conv_bias_std=1.0)
    with pytest.raises(NotImplementedError, match="alpha-only BaB does not yet support conv graphs"):
        bab_ref.solve_bab_mlp(w.module, w.spec, linear_spec_C=w.C, config={**DEFAULTS, "oracle": "alpha"})
