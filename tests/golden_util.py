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
    "bab_solve_obj_both": (dict(eps=0.05), dict(max_nodes=40, oracle="alpha_beta", node_batch_size=8, alpha_steps=10,
                                                objective="both", spec_reduce="softmin", soft_tau=0.5,
                                                ub_weight=0.5)),
    "bab_solve_obj_alpha_gap": (dict(eps=0.05), dict(max_nodes=20, oracle="alpha", node_batch_size=1,
                                                     alpha_steps=10, objective="gap", spec_reduce="min")),
    # conv graphs (make_bab_cnn_toy: conv 2x6x6 -> 2x4x4, fc 16, fc 3).  Each example has at most
    # one ambiguous first-layer (conv) neuron, so a node carries at most one first-layer split:
    # the reference's certificate evaluates the conv row's halfspace (alpha_beta_crown.py:345-389)
    # and does not reach its multi-halfspace stack, which cannot broadcast conv rows.
    "bab_solve_cnn_b1": (dict(kind="cnn", seed=2, eps=0.01, channels=2, hidden=16, conv_bias_std=1.0),
                         dict(max_nodes=30, oracle="alpha_beta", node_batch_size=1, alpha_steps=5)),
    "bab_solve_cnn_b4": (dict(kind="cnn", seed=4, eps=0.02, channels=2, hidden=16, conv_bias_std=1.0),
                         dict(max_nodes=30, oracle="alpha_beta", node_batch_size=4, alpha_steps=5)),
}


# run_alpha_beta_crown_mlp options of the "objectives_mlp" fixture (objective, spec reduction,
# temperature, weights, per-domain or shared parameters); alpha_beta_crown.py:756-815
OBJECTIVE_CASES = {
    "upper_mean": dict(objective="upper", spec_reduce="mean", per_batch_params=True),
    "gap_min": dict(objective="gap", spec_reduce="min", per_batch_params=True),
    "both_softmin": dict(objective="both", spec_reduce="softmin", soft_tau=0.5, lb_weight=1.0, ub_weight=0.5,
                         per_batch_params=True),
    "lower_min": dict(objective="lower", spec_reduce="min", per_batch_params=True),
    "lower_softmin": dict(objective="lower", spec_reduce="softmin", soft_tau=2.0, per_batch_params=True),
    "gap_mean_shared": dict(objective="gap", spec_reduce="mean", per_batch_params=False),
}


# run_alpha_crown_mlp options of the "alpha_crown_objectives" fixture (shared alpha);
# alpha_crown.py:62-135
ALPHA_CROWN_OBJECTIVE_CASES = {
    "upper_mean": dict(objective="upper", spec_reduce="mean"),
    "gap_min": dict(objective="gap", spec_reduce="min"),
    "both_softmin": dict(objective="both", spec_reduce="softmin", soft_tau=0.5, lb_weight=1.0, ub_weight=0.5),
    "lower_softmin": dict(objective="lower", spec_reduce="softmin", soft_tau=2.0),
}


def objective_workload():
    """The "objectives_mlp" problem: make_bab_toy(seed 4, eps 0.1, 12-16-16-4, 6 inputs) with
    feasible random splits, chosen layer by layer among the neurons still ambiguous
    after the splits of the layers before (about one in five, random sign)."""
    import torch

    from boundflow_amd import workloads as wl
    from oracle import crown_ref as cr

    w = wl.make_bab_toy(seed=4, eps=0.1, dims=(12, 16, 16, 4), batch=6)
    g = torch.Generator().manual_seed(6)
    names = [op.inputs[0] for op in w.module.get_entry_task().ops if op.op_type == "relu"]
    splits = {n: torch.zeros(6, 16, dtype=torch.int8) for n in names}
    for n in names:
        _env, pre = cr.forward_ibp_trace(w.module, w.spec, relu_split_state=splits)
        amb = (pre[n].lower < 0) & (pre[n].upper > 0)
        pick = amb & (torch.rand(6, 16, generator=g) < 0.2)
        sign = (torch.randint(0, 2, (6, 16), generator=g) * 2 - 1).to(torch.int8)
        splits[n] = torch.where(pick, sign, splits[n])
    return w, splits


def c3_box(batch: int = 6):
    """The C3 CNN on a box input: the first ``batch`` C3 inputs widened by 0.01 and
    clipped to [0, 1] (fixture crown_c3_box)."""
    from boundflow_amd import workloads as wl
    from boundflow_amd.spec import InputSpec
    w = wl.subset(wl.make_c3(), batch)
    lo = (w.spec.center - 0.01).clamp(0, 1)
    hi = (w.spec.center + 0.01).clamp(0, 1)
    return wl.Workload("C3box", w.module, InputSpec.box(value_name="input", lower=lo, upper=hi), w.C, w.labels)


def dag_case(kind: str, box: bool):
    """The DAG workload of fixture crown_dag_<kind>[_box]."""
    from boundflow_amd import workloads as wl
    return wl.make_dag(kind, seed=3, batch=6, eps=0.03, box=box, blocks=2)


# L2 / L1 input balls (LpBallPerturbation p=2, p=1): radii that leave a mix of stable and
# unstable ReLUs on each network, shared by the reference fixtures (lp_reference_p{p}) and
# the tests that read them
LP_EPS = {"mlp": {2: 0.3, 1: 1.0}, "cnn": {2: 0.02, 1: 0.03}, "dag": {2: 0.08, 1: 0.2}, "c5": {2: 0.1, 1: 0.5},
          "c4": {2: 0.01, 1: 0.01}, "cert_c5": {2: 0.5, 1: 2.0}}
# whole searches over the balls: (eps, BabConfig options) per p
LP_BAB = {2: (0.1, dict(max_nodes=40, oracle="alpha_beta", node_batch_size=8, alpha_steps=10)),
          1: (0.25, dict(max_nodes=20, oracle="alpha", node_batch_size=1, alpha_steps=10))}


def lp_workload(w, p, eps, C=None):
    """The workload ``w`` with its input set replaced by the Lp ball of radius eps at its centers."""
    from boundflow_amd import workloads as wl
    from boundflow_amd.spec import InputSpec, LpBallPerturbation
    spec = InputSpec(value_name=w.spec.value_name, center=w.spec.center,
                     perturbation=LpBallPerturbation(p=p, eps=eps))
    return wl.Workload(w.name, w.module, spec, w.C if C is None else C, w.labels, {})


def lp_case(kind: str, p: int):
    """The networks of the Lp reference fixtures: "mlp" (C1, 16 inputs), "cnn" (C3, 8
    inputs), "alpha" (C1, 8 inputs: alpha-CROWN from CROWN slopes, 10 steps, lr 0.1),
    "cert_c5" (the C5 network, 48 domains, first-layer certificate) and "bab" (a residual
    MLP of 4 inputs for whole searches)."""
    from boundflow_amd import workloads as wl
    if kind == "mlp":
        return lp_workload(wl.make_c1(batch=16), p, LP_EPS["mlp"][p])
    if kind == "cnn":
        return lp_workload(wl.make_c3(batch=8), p, LP_EPS["cnn"][p])
    if kind == "alpha":
        return lp_workload(wl.make_c1(batch=8), p, LP_EPS["mlp"][p])
    if kind == "cert_c5":
        return lp_workload(wl.make_c5(domains=48), p, LP_EPS["cert_c5"][p])
    if kind == "bab":
        base = wl.make_dag("residual_mlp", seed=12, batch=4, eps=0.03, n_in=8, hidden=12, n_out=4, blocks=1)
        return lp_workload(base, p, LP_BAB[p][0])
    raise ValueError(kind)


def lp_cert_nodes(w, p):
    """48 first-layer split rows on the C5 network's ambiguous neurons (2-12 per node)."""
    from oracle import crown_ref as cr
    from boundflow_amd import workloads as wl
    g = torch.Generator().manual_seed(4 + p)
    _env, pre = cr.forward_ibp_trace(w.module, wl.subset(w, 1).spec)
    name = next(iter(pre))
    l, u = pre[name].lower[0], pre[name].upper[0]
    amb = ((l < 0) & (u > 0)).nonzero().flatten()
    rows = torch.zeros(48, int(l.numel()), dtype=torch.int8)
    for r in range(48):
        k = int(torch.randint(2, 13, (1,), generator=g))
        pick = amb[torch.randperm(int(amb.numel()), generator=g)[:k]]
        rows[r, pick] = (torch.randint(0, 2, (int(pick.numel()),), generator=g) * 2 - 1).to(torch.int8)
    return name, rows

