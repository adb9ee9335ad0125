"""Helpers to load the committed golden fixtures (numpy, no pickle)."""

import hashlib
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name: str):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def workload_checksum(w) -> str:
    h = hashlib.sha256()
    ts = [w.spec.center, w.C] + [w.module.params[k] for k in sorted(w.module.params)]
    if "splits" in w.extra:
        ts += [w.extra["splits"][k] for k in sorted(w.extra["splits"])]
    for t in ts:
        h.update(t.detach().cpu().contiguous().numpy().tobytes())
    return h.hexdigest()


def t(x):
    return torch.from_numpy(np.asarray(x))


# Whole branch-and-bound searches of the reference's solve_bab_mlp (fixtures written by
# tests/golden/make_golden.py): tag -> (make_bab_toy arguments, BabConfig fields).  The
# "cert" cases are searches in which the first-layer split certificate
# (alpha_beta_crown.py:391-532) closes nodes: node by node (node_batch_size 1), through
# the per-node fallback of a node batch holding an IBP-infeasible node
# (bab.py:1399-1456), and as pre-pruning (enable_batch_infeasible_prune, bab.py:373-425);
# "1d" narrows a one-input network's Linf interval by the first-layer splits
# (bab.py:524-628).
BAB_SOLVE_CASES = {
    "bab_solve_ab_e003": (dict(eps=0.03), dict(max_nodes=40, oracle="alpha_beta", node_batch_size=8, alpha_steps=10)),
    "bab_solve_ab_e005": (dict(eps=0.05), dict(max_nodes=40, oracle="alpha_beta", node_batch_size=8, alpha_steps=10)),
    "bab_solve_alpha_e005": (dict(eps=0.05), dict(max_nodes=20, oracle="alpha", node_batch_size=1, alpha_steps=10)),
    "bab_solve_cert_single": (dict(seed=2, eps=0.1, dims=(6, 8, 8, 3), batch=4),
                              dict(max_nodes=30, oracle="alpha_beta", node_batch_size=1, alpha_steps=5)),
    "bab_solve_cert_fallback": (dict(seed=8, eps=0.1, dims=(3, 10, 8, 3), batch=4),
                                dict(max_nodes=30, oracle="alpha_beta", node_batch_size=4, alpha_steps=5)),
    "bab_solve_cert_prune": (dict(seed=8, eps=0.1, dims=(3, 10, 8, 3), batch=4),
                             dict(max_nodes=30, oracle="alpha_beta", node_batch_size=4, alpha_steps=5,
                                  enable_batch_infeasible_prune=True)),
    "bab_solve_1d": (dict(seed=3, eps=0.4, dims=(1, 8, 8, 2), batch=4),
                     dict(max_nodes=30, oracle="alpha_beta", node_batch_size=4, alpha_steps=5,
                          use_1d_linf_input_restriction_patch=True)),
}
