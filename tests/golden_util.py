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
