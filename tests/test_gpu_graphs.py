"""HIP graph replay of launch-bound queries (boundflow_amd.graphs).

Every replay must reproduce the eager result exactly: the same kernels run on
the same buffers.  Replays are interleaved with unrelated eager work and host
synchronizations, and each one is checked, as graph replays after the first
are where recorded memset nodes have gone wrong on this hardware.
"""

import pytest
import torch

from boundflow_amd import alpha_beta as hab
from boundflow_amd import bab as hbab
from boundflow_amd import crown as hc
from boundflow_amd import graphs
from boundflow_amd import workloads as wl
from tests.gpu_util import announce, device

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,n", [("C1", 64), ("C3", 16)])
def test_captured_query_replays_match_eager(name, n):
    dev = device()
    announce(f"graph replay of run_crown_ibp_mlp {name} (batch {n})")
    wd = wl.to_device(wl.subset(wl.make(name), n), dev)
    eager = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
    torch.cuda.synchronize()
    ref_lo, ref_hi = eager.lower.clone(), eager.upper.clone()
    cap = graphs.CapturedQuery(lambda: hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C))
    for rep in range(4):
        # unrelated eager work between replays
        junk = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
        junk.lower.add_(1.0)
        torch.cuda.synchronize()
        out = cap()
        torch.cuda.synchronize()
        assert torch.equal(out.lower, ref_lo), f"replay {rep} lower"
        assert torch.equal(out.upper, ref_hi), f"replay {rep} upper"


def test_captured_alpha_crown_replays_match_eager():
    """The whole C4 query: forward trace, alpha from CROWN, 20 Adam steps with
    best-of tracking -- no host synchronization, so one graph."""
    dev = device()
    announce("graph replay of run_alpha_crown_from_crown_init (C4, batch 4)")
    wd = wl.to_device(wl.subset(wl.make_c4(), 4), dev)

    def query():
        return hab.run_alpha_crown_from_crown_init(wd.module, wd.spec, linear_spec_C=wd.C, steps=20, lr=0.1)[0]

    eager = query()
    torch.cuda.synchronize()
    ref_lo, ref_hi = eager.lower.clone(), eager.upper.clone()
    cap = graphs.CapturedQuery(query)
    for rep in range(3):
        junk = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
        junk.lower.add_(1.0)
        torch.cuda.synchronize()
        out = cap()
        torch.cuda.synchronize()
        assert torch.equal(out.lower, ref_lo), f"replay {rep} lower"
        assert torch.equal(out.upper, ref_hi), f"replay {rep} upper"


def test_captured_domain_batch_replays_match_eager():
    """A C5 domain batch (splits, 10 alpha-beta steps, certification) has no host
    synchronization either: every replay gives the eager statuses, bounds and
    branching decisions."""
    dev = device()
    announce("graph replay of evaluate_domain_batch (C5, 256 domains)")
    wd = wl.to_device(wl.subset(wl.make_c5(), 256), dev)

    def batch():
        return hbab.evaluate_domain_batch(wd.module, wd.spec, linear_spec_C=wd.C,
                                          relu_split_state=wd.extra["splits"], steps=10, lr=0.2)

    eager = batch()
    torch.cuda.synchronize()
    keys = ("status", "lower", "upper", "branch_layer", "branch_neuron")
    ref = {k: eager[k].clone() for k in keys}
    cap = graphs.CapturedQuery(batch)
    for rep in range(3):
        junk = batch()
        junk["lower"].add_(1.0)
        torch.cuda.synchronize()
        out = cap()
        torch.cuda.synchronize()
        for k in keys:
            assert torch.equal(out[k], ref[k]), f"replay {rep} {k}"


def test_replay_sees_inputs_and_parameters_changed_in_place():
    """A captured C1 query (box input) after ``copy_`` of a different box into the
    perturbation and an in-place change of a layer weight: the replay recomputes
    the box radius inside the graph, and the weight transposes the graph reads
    (kept by the captured query, not by the process-wide cache) are remade in
    place before the replay, so it equals an eager query on the new values."""
    dev = device()
    announce("graph replay after in-place input and parameter updates (C1, batch 16)")
    wd = wl.to_device(wl.subset(wl.make_c1(), 16), dev)
    hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)   # fills the parameter cache
    cap = graphs.CapturedQuery(lambda: hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C))
    pert = wd.spec.perturbation
    lo0, hi0 = pert.lower.clone(), pert.upper.clone()
    W1 = wd.module.params["W1"]
    W1_0 = W1.clone()
    for rep, (shrink, wscale) in enumerate([(0.5, 1.0), (0.25, 0.9), (1.0, 1.0)]):
        mid = (lo0 + hi0) / 2
        rad = (hi0 - lo0) / 2 * shrink
        pert.lower.copy_(mid - rad)
        pert.upper.copy_(mid + rad)
        W1.copy_(W1_0 * wscale)
        torch.cuda.synchronize()
        out = cap()
        torch.cuda.synchronize()
        got_lo, got_hi = out.lower.clone(), out.upper.clone()
        eager = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
        torch.cuda.synchronize()
        assert torch.equal(got_lo, eager.lower), f"replay {rep} lower"
        assert torch.equal(got_hi, eager.upper), f"replay {rep} upper"
