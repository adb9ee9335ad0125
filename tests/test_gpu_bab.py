"""HIP branch and bound (boundflow_amd.bab.solve_bab_mlp) against whole
searches of the reference's solve_bab_mlp (tests/golden) on small BaB
workloads, including searches where the first-layer split certificate closes
nodes (node by node, in the per-node fallback of a batch, as pre-pruning) and a
one-input network under the 1-D input restriction: identical statuses, node
counts, rounds and queue size (every certification, infeasibility and
branching decision matches); best bounds within rtol 1e-4 (the count outside
the 1e-5 / 1e-6 contract is reported: they end 5- and 10-step Adam
trajectories)."""

import numpy as np
import pytest
import torch

from boundflow_amd import bab as hbab
from boundflow_amd import workloads as wl
from tests.golden_util import BAB_SOLVE_CASES, load
from tests.gpu_util import announce, device

pytestmark = pytest.mark.gpu

CASES = BAB_SOLVE_CASES
CODE = {"proven": 0, "unsafe": 1, "unknown": 2}


@pytest.mark.parametrize("tag", list(CASES))
def test_hip_bab_search_matches_reference(tag):
    dev = device()
    toy, kw = CASES[tag]
    announce(f"solve_bab_mlp {tag}")
    g = load(tag)
    wd = wl.to_device(wl.make_bab_case(**toy), dev)
    r = hbab.solve_bab_mlp(wd.module, wd.spec, linear_spec_C=wd.C, config=hbab.BabConfig(**kw))
    per = r.per_example
    announce(f"  statuses {[p.status for p in per]} visited {[p.nodes_visited for p in per]} "
             f"rounds {r.batch_rounds}")
    assert CODE[r.status] == int(g["status"])
    assert [CODE[p.status] for p in per] == g["per_status"].tolist()
    assert [p.nodes_visited for p in per] == g["per_visited"].tolist()
    assert [p.nodes_evaluated for p in per] == g["per_evaluated"].tolist()
    assert [p.nodes_expanded for p in per] == g["per_expanded"].tolist()
    assert (r.max_queue, r.batch_rounds) == (int(g["max_queue"]), int(g["batch_rounds"]))
    assert abs(r.avg_batch_fill_rate - float(g["avg_batch_fill_rate"])) < 1e-12
    got = np.array([[p.best_lower for p in per], [p.best_upper for p in per]])
    ref = np.stack([g["per_best_lower"], g["per_best_upper"]])
    finite = np.isfinite(ref)
    d = np.abs(got - ref)[finite]
    out = int((d > 1e-6 + 1e-5 * np.abs(ref[finite])).sum())
    announce(f"  best bounds: max abs diff {d.max() if d.size else 0.0:.3e}, outside 1e-5/1e-6: {out}/{d.size}")
    assert np.array_equal(np.isfinite(got), finite)
    np.testing.assert_allclose(got[finite], ref[finite], rtol=1e-4, atol=1e-5)


def test_hip_bab_frontier_growth_and_budget():
    """A budget far below the tree size: the frontier grows past its initial
    capacity and every example ends "unknown" or decided, never open."""
    dev = device()
    announce("solve_bab_mlp frontier growth")
    wd = wl.to_device(wl.make_bab_toy(eps=0.12, batch=6), dev)
    r = hbab.solve_bab_mlp(wd.module, wd.spec, linear_spec_C=wd.C,
                           config=hbab.BabConfig(max_nodes=60, oracle="alpha_beta", node_batch_size=16,
                                                 alpha_steps=4))
    assert all(p.status in ("proven", "unsafe", "unknown") for p in r.per_example)
    assert all(p.nodes_visited <= 60 for p in r.per_example)
    assert r.max_queue >= 1 and r.batch_rounds >= 1


def test_alpha_oracle_refuses_conv_graphs():
    """The reference's alpha-only BaB does not take conv graphs (bab.py:656-659)."""
    dev = device()
    announce("solve_bab_mlp alpha oracle on a conv graph")
    wd = wl.to_device(wl.make_bab_cnn_toy(seed=2, eps=0.01, channels=2, hidden=16, conv_bias_std=1.0), dev)
    with pytest.raises(NotImplementedError, match="alpha-only BaB does not yet support conv graphs"):
        hbab.solve_bab_mlp(wd.module, wd.spec, linear_spec_C=wd.C, config=hbab.BabConfig(oracle="alpha"))
