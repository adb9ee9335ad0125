"""Parity at the BASELINE configurations' full sizes, against the CPU oracle run
on the same seeded inputs.

* C2 (CROWN with every intermediate bound by CROWN, B = 256) and C3 (CROWN CNN,
  B = 128): both bounds at the contract (|hip - ref| <= 1e-6 + 1e-5 |ref|), or
  fp64-explained; identical verdicts except near-ties.
* C4 (alpha-CROWN, B = 32, 20 Adam steps) and C5 (beta-CROWN domain batch,
  4096 domains, 10 steps): whole trajectories.  Identical verdicts (C4) and,
  over all 4096 domains, identical feasibility, certified flags, certified /
  remaining counts and branching decisions (C5).  The optimised bounds end Adam
  trajectories that amplify fp32 rounding (one step at a time they meet the
  contract, tests/test_gpu_teacher_forced.py): the counts outside the contract
  and outside 1e-4 (with fp64 explanation) are reported, and every bound must lie
  within the trajectory band TRAJ_RTOL / TRAJ_ATOL of the reference or be
  fp64-explained there."""

import pytest
import torch

from boundflow_amd import alpha_beta as hab
from boundflow_amd import bab as hbab
from boundflow_amd import crown as hc
from boundflow_amd import workloads as wl
from oracle import alpha_beta_ref as ab
from oracle import crown_ref as cr
from oracle import parity
from tests.gpu_util import announce, assert_verdicts, device

pytestmark = pytest.mark.gpu


def _contract(got, ref32, what, ref64_fn):
    rep = parity.compare(got, ref32, None)
    if rep.strict_violations:
        rep = parity.compare(got, ref32, ref64_fn())
    announce(rep.line(what))
    assert rep.ok, rep.line(what)
    return rep


def test_c2_full_size():
    dev = device()
    announce("full-size C2: CROWN all-intermediate, MLP 784-500x6-10, B=256")
    torch.set_num_threads(max(1, torch.get_num_threads()))
    w = wl.make_c2()
    wd = wl.to_device(w, dev)
    got, _pre = hc.run_crown_all_intermediate(wd.module, wd.spec, linear_spec_C=wd.C)
    torch.cuda.synchronize()
    with torch.inference_mode():
        ref, _ = cr.run_crown_all_intermediate(w.module, w.spec, linear_spec_C=w.C)
    cache = {}

    def ref64():
        if "r" not in cache:
            w64 = parity.to_float64(w)
            with torch.inference_mode():
                cache["r"] = cr.run_crown_all_intermediate(w64.module, w64.spec, linear_spec_C=w64.C)[0]
        return cache["r"]

    _contract(got.lower, ref.lower, "C2 full lower", lambda: ref64().lower)
    _contract(got.upper, ref.upper, "C2 full upper", lambda: ref64().upper)
    assert_verdicts(got.lower, ref.lower, ref64().lower if cache else None, "C2 full")


def test_c3_full_size():
    dev = device()
    announce("full-size C3: CROWN CNN, B=128")
    w = wl.make_c3()
    wd = wl.to_device(w, dev)
    got = hc.run_crown_ibp_mlp(wd.module, wd.spec, linear_spec_C=wd.C)
    torch.cuda.synchronize()
    with torch.inference_mode():
        ref = cr.run_crown_ibp(w.module, w.spec, linear_spec_C=w.C)
    w64 = parity.to_float64(w)
    with torch.inference_mode():
        ref64 = cr.run_crown_ibp(w64.module, w64.spec, linear_spec_C=w64.C)
    _contract(got.lower, ref.lower, "C3 full lower", lambda: ref64.lower)
    _contract(got.upper, ref.upper, "C3 full upper", lambda: ref64.upper)
    assert_verdicts(got.lower, ref.lower, ref64.lower, "C3 full")


# Band of a whole optimisation trajectory: 100x the contract.  One step meets the
# contract (tests/test_gpu_teacher_forced.py); over 10-20 steps, gradients whose sign
# is decided by fp32 rounding (input-layer coefficients within rounding of zero) move
# Adam's normalised step by up to lr, and the trajectories part by that much.
TRAJ_RTOL = TRAJ_ATOL = 1e-3


def _trajectory_report(got, ref32, ref64_fn, what):
    """Counts at the contract and at 1e-4 (fp64-explained), asserted at the trajectory band."""
    strict = parity.compare(got, ref32, None)
    announce(f"{what}: at the contract 1e-5/1e-6: {strict.strict_violations}/{strict.n} outside "
             f"(max_abs {strict.max_abs:.3e}, max_rel {strict.max_rel:.3e})")
    ref64 = ref64_fn() if strict.strict_violations else None
    mid = parity.compare(got, ref32, ref64, rtol=1e-4, atol=1e-4)
    announce(mid.line(f"{what} at 1e-4"))
    band = parity.compare(got, ref32, ref64, rtol=TRAJ_RTOL, atol=TRAJ_ATOL)
    announce(band.line(f"{what} at the trajectory band {TRAJ_RTOL:g}"))
    assert band.ok, band.line(what)


def test_c4_full_size_trajectory():
    dev = device()
    announce("full-size C4: alpha-CROWN CNN, B=32, 20 Adam steps, lr 0.1, alpha from CROWN")
    w = wl.make_c4()
    wd = wl.to_device(w, dev)
    got, _a, _b, _st = hab.run_alpha_crown_from_crown_init(wd.module, wd.spec, linear_spec_C=wd.C, steps=20, lr=0.1)
    torch.cuda.synchronize()
    _e, pre = cr.forward_ibp_trace(w.module, w.spec)
    ref, _ra, _rb, _ch = ab.run_alpha_beta_crown(w.module, w.spec, linear_spec_C=w.C, steps=20, lr=0.1,
                                                 warm_start_alpha=ab.adaptive_alpha_init(pre), per_batch_params=True)
    cache = {}

    def ref64():
        if "r" not in cache:
            w64 = parity.to_float64(w)
            _e64, pre64 = cr.forward_ibp_trace(w64.module, w64.spec)
            cache["r"] = ab.run_alpha_beta_crown(w64.module, w64.spec, linear_spec_C=w64.C, steps=20, lr=0.1,
                                                 warm_start_alpha=ab.adaptive_alpha_init(pre64),
                                                 per_batch_params=True)[0]
        return cache["r"]

    _trajectory_report(got.lower, ref.lower, lambda: ref64().lower, "C4 full lower")
    _trajectory_report(got.upper, ref.upper, lambda: ref64().upper, "C4 full upper")
    assert_verdicts(got.lower, ref.lower, ref64().lower, "C4 full")


def test_c5_full_size_domain_batch():
    dev = device()
    announce("full-size C5: beta-CROWN domain batch, 4096 domains, 10 steps, lr 0.2")
    w = wl.make_c5()
    wd = wl.to_device(w, dev)
    r = hbab.evaluate_domain_batch(wd.module, wd.spec, linear_spec_C=wd.C, relu_split_state=wd.extra["splits"],
                                   steps=10, lr=0.2)
    status = r["status"].cpu()
    ref = ab.evaluate_domain_batch(w.module, w.spec, linear_spec_C=w.C, relu_split_state=w.extra["splits"],
                                   steps=10, lr=0.2)
    feasible = status != 2
    assert torch.equal(feasible, ref["feasible"]), "feasibility flags differ"
    certified = status == 1
    n_cert, n_ref = int(certified.sum()), int(ref["certified"].sum())
    announce(f"C5 full: certified hip {n_cert} / ref {n_ref}; remaining hip {int(feasible.sum()) - n_cert} / ref "
             f"{int(ref['feasible'].sum()) - n_ref}; infeasible {int((~feasible).sum())}")
    names = r["relu_names"]
    layer = r["branch_layer"].cpu().tolist()
    neuron = r["branch_neuron"].cpu().tolist()
    hip_branch = [None if l < 0 else (names[l], n) for l, n in zip(layer, neuron)]
    mism = [i for i in range(len(hip_branch)) if bool(ref["feasible"][i]) and hip_branch[i] != ref["branch"][i]]
    announce(f"C5 full: branch decisions identical on {int(feasible.sum()) - len(mism)}/{int(feasible.sum())}")
    assert not mism, f"branch decisions differ at {mism[:10]}"
    lo = r["lower"].cpu()[feasible]
    ref_lo = ref["lower"][feasible]
    cache = {}

    def ref64():
        if "r" not in cache:
            w64 = parity.to_float64(w)
            cache["r"] = ab.evaluate_domain_batch(w64.module, w64.spec, linear_spec_C=w64.C,
                                                  relu_split_state=w64.extra["splits"], steps=10, lr=0.2)
        return cache["r"]["lower"][feasible]

    _trajectory_report(lo, ref_lo, ref64, "C5 full lower")
    mism_v, flips, ties = parity.verdict_parity(lo, ref_lo, None)
    announce(f"C5 full: certified flags differ on {int((certified != ref['certified']).sum())} domains "
             f"(near-ties {ties})")
    assert torch.equal(certified, ref["certified"]), "certified flags differ"
