"""Build the HIP library in-tree: boundflow_amd/libboundflow_hip.so (gfx950).

Usage: python -m boundflow_amd.build   (or boundflow_amd.build.build())
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libboundflow_hip.so"
SOURCES = ["bf_gemm.hip", "bf_ops.hip", "bf_conv.hip", "bf_grad.hip"]
ARCH = os.environ.get("BOUNDFLOW_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False) -> Path:
    srcs = [str(CSRC / s) for s in SOURCES if (CSRC / s).exists()]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # no implicit a*b+c fusion: elementwise steps round like the CPU oracle's separate ops
        "-ffp-contract=off",
        "-Wno-unused-command-line-argument",
        f"-I{CSRC}", "-o", str(tmp), *srcs,
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    print("built", LIB, file=sys.stderr)
