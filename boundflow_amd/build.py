"""Build the HIP library in-tree: boundflow_amd/libboundflow_hip.so (gfx950).

Usage: python -m boundflow_amd.build   (or boundflow_amd.build.build())
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libboundflow_hip.so"
ARCH = os.environ.get("BOUNDFLOW_OFFLOAD_ARCH", "gfx950")
# no implicit a*b+c fusion: elementwise steps round like the CPU oracle's separate ops
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-ffp-contract=off", "-Wno-unused-command-line-argument"]
NOISE = "is not a recognized feature for this target"


def sources() -> list:
    """Every HIP translation unit of the library (one per contraction tile configuration among them)."""
    return sorted(str(p) for p in CSRC.glob("*.hip"))


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _clean(stderr: str) -> str:
    return "\n".join(l for l in stderr.splitlines() if NOISE not in l)


def build(verbose: bool = False, jobs: int = 0) -> Path:
    """Compile every source to an object (in parallel), then link the shared library."""
    cc = hipcc()
    jobs = jobs or max(1, min(os.cpu_count() or 1, 16))
    with tempfile.TemporaryDirectory(prefix="bf_build_") as tmpdir:
        pending = [(src, str(Path(tmpdir) / (Path(src).stem + ".o"))) for src in sources()]
        running, objs = [], []
        while pending or running:
            while pending and len(running) < jobs:
                src, obj = pending.pop(0)
                cmd = [cc, f"--offload-arch={ARCH}", *FLAGS, f"-I{CSRC}", "-c", src, "-o", obj]
                if verbose:
                    print(" ".join(cmd), flush=True)
                running.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
                objs.append(obj)
            src, proc = running.pop(0)
            _, err = proc.communicate()
            err = _clean(err)
            if proc.returncode != 0:
                for _, other in running:
                    other.kill()
                    other.wait()
                raise RuntimeError(f"hipcc failed on {src} ({proc.returncode}):\n{err}")
            if err.strip() and verbose:
                print(err, file=sys.stderr)
        tmp = LIB.with_suffix(".so.tmp")
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed ({res.returncode}):\n{_clean(res.stderr)}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    print("built", LIB, file=sys.stderr)
