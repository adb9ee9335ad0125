"""Parity at the BASELINE configurations' full sizes, against the CPU oracle run
on the same seeded inputs.

* C2 (CROWN with every intermediate bound by CROWN, B = 256) and C3 (CROWN CNN,
  B = 128): both bounds at the contract (|hip - ref| <= 1e-6 + 1e-5 |ref|), or
  fp64-explained; identical verdicts except near-ties.
* C4 (alpha-CROWN, B = 32, 20 Adam steps) and C5 (beta-CROWN domain batch,
  4096 domains, 10 steps; the BASELINE batch, where no domain certifies, and a
  batch of the same network at eps 3e-5 with the predicted label, where about
  half do): identical verdicts (C4) and, over all 4096 domains, identical
  feasibility, certified flags, certified / remaining counts and branching
  decisions (C5).  The optimised bounds are held to the contract with no band:
  a domain with a bound outside it is traced (oracle/trajectory.py) -- the HIP
  path's own recorded trajectory is checked step by step against the oracle
  evaluated at the HIP states (bounds, gradients within their fp32 uncertainty
  or a computed kink allowance, the Adam update), and the first step at which
  the HIP and oracle parameters part is shown to be one that Adam reaches from
  the oracle's state within the gradients' fp32 uncertainty.  A sample of
  in-contract domains is shadow-checked the same way."""

import pytest
import torch

from boundflow_amd import alpha_beta as hab
from boundflow_amd import bab as hbab
from boundflow_amd import crown as hc
from boundflow_amd import workloads as wl
from oracle import alpha_beta_ref as ab
from oracle import crown_ref as cr
from oracle import parity
from oracle import trajectory as tt
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


def test_c4_full_size_trajectory():
    dev = device()
    announce("full-size C4: alpha-CROWN CNN, B=32, 20 Adam steps, lr 0.1, alpha from CROWN")
    w = wl.make_c4()
    wd = wl.to_device(w, dev)
    hrec = []
    got, best_alpha, _b, _st = hab.run_alpha_crown_from_crown_init(wd.module, wd.spec, linear_spec_C=wd.C, steps=20,
                                                                   lr=0.1, record=hrec)
    torch.cuda.synchronize()
    _e, pre = cr.forward_ibp_trace(w.module, w.spec)
    srec = []
    ref = ab.run_alpha_beta_crown(w.module, w.spec, linear_spec_C=w.C, steps=20, lr=0.1,
                                  warm_start_alpha=ab.adaptive_alpha_init(pre), per_batch_params=True,
                                  record=srec)[0]

    def fp64_lower(rows):
        w64 = parity.to_float64(tt.sub_workload(w, rows))
        _e64, pre64 = cr.forward_ibp_trace(w64.module, w64.spec)
        return ab.run_alpha_beta_crown(w64.module, w64.spec, linear_spec_C=w64.C, steps=20, lr=0.1,
                                       warm_start_alpha=ab.adaptive_alpha_init(pre64), per_batch_params=True)[0].lower

    summary = tt.trace_run(w, hrec, srec, got.lower.cpu(), ref.lower, 0.1, what="C4 full", sample=range(w.batch),
                           got_upper=got.upper.cpu(), ref_upper=ref.upper,
                           best_alpha={n: v.cpu() for n, v in best_alpha.items()}, fp64_lower=fp64_lower,
                           log=announce)
    announce(f"C4 full trace: {summary}")
    assert_verdicts(got.lower, ref.lower, None, "C4 full")


@pytest.mark.parametrize("variant", ["baseline", "certifying"])
def test_c5_full_size_domain_batch(variant):
    """baseline: the BASELINE C5 batch (eps 0.03, random label; no domain certifies on
    either side).  certifying: the same network and split generator at eps 3e-5 with
    the predicted label, where about half the domains certify, so that the certified /
    remaining counts and statuses compare real verdicts."""
    dev = device()
    announce(f"full-size C5 ({variant}): beta-CROWN domain batch, 4096 domains, 10 steps, lr 0.2")
    w = wl.make_c5() if variant == "baseline" else wl.make_c5(eps=3e-5, label_mode="predicted")
    wd = wl.to_device(w, dev)
    hrec = []
    r = hbab.evaluate_domain_batch(wd.module, wd.spec, linear_spec_C=wd.C, relu_split_state=wd.extra["splits"],
                                   steps=10, lr=0.2, record=hrec)
    status = r["status"].cpu()
    srec = []
    ref = ab.evaluate_domain_batch(w.module, w.spec, linear_spec_C=w.C, relu_split_state=w.extra["splits"],
                                   steps=10, lr=0.2, record=srec)
    feasible = status != 2
    assert torch.equal(feasible, ref["feasible"]), "feasibility flags differ"
    certified = status == 1
    n_cert, n_ref = int(certified.sum()), int(ref["certified"].sum())
    announce(f"C5 {variant}: certified hip {n_cert} / ref {n_ref}; remaining hip {int(feasible.sum()) - n_cert} / "
             f"ref {int(ref['feasible'].sum()) - n_ref}; infeasible {int((~feasible).sum())}")
    assert n_cert == n_ref, "certified counts differ"
    assert torch.equal(certified, ref["certified"]), "certified flags differ"
    if variant == "certifying":
        assert 0.2 * w.batch <= n_ref <= 0.8 * w.batch, f"the certifying batch certifies {n_ref} of {w.batch}"
    names = r["relu_names"]
    layer = r["branch_layer"].cpu().tolist()
    neuron = r["branch_neuron"].cpu().tolist()
    hip_branch = [None if l < 0 else (names[l], n) for l, n in zip(layer, neuron)]
    mism = [i for i in range(len(hip_branch)) if bool(ref["feasible"][i]) and hip_branch[i] != ref["branch"][i]]
    announce(f"C5 {variant}: branch decisions identical on {int(feasible.sum()) - len(mism)}/{int(feasible.sum())}")
    assert not mism, f"branch decisions differ at {mism[:10]}"
    idx = feasible.nonzero().flatten()
    wf = tt.sub_workload(w, idx)
    hrec_f = tt.slice_record(hrec, idx)

    def fp64_lower(rows):
        w64 = parity.to_float64(tt.sub_workload(wf, rows))
        return ab.run_alpha_beta_crown(w64.module, w64.spec, linear_spec_C=w64.C,
                                       relu_split_state=w64.extra["splits"], steps=10, lr=0.2,
                                       per_batch_params=True)[0].lower

    best_alpha = {n: v.cpu()[idx] for n, v in r["alpha"].items()}
    summary = tt.trace_run(wf, hrec_f, srec, r["lower"].cpu()[idx], ref["lower"][idx], 0.2, what=f"C5 {variant}",
                           sample=range(0, len(idx), 64), got_upper=r["upper"].cpu()[idx], ref_upper=None,
                           best_alpha=best_alpha, fp64_lower=fp64_lower, log=announce)
    announce(f"C5 {variant} trace: {summary}")
