"""The C ABI: the header compiles as plain C, and the built library exports
exactly the entry points the header declares and the Python binding uses.
No device call is made (runs without a GPU)."""

import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "boundflow_hip.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(bf_[a-z0-9_]+)\s*\(", text)))


def test_header_compiles_as_c():
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "t.c")
        with open(src, "w") as f:
            f.write('#include "boundflow_hip.h"\nint (*probe)(void) = bf_abi_version;\n')
        subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-c", "-I", os.path.dirname(HEADER), src, "-o",
                        os.path.join(d, "t.o")], check=True)


def test_binding_matches_header():
    from boundflow_amd import _lib
    assert sorted(_lib.SIGNATURES) == header_symbols()


def test_library_exports_every_declared_symbol():
    from boundflow_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built (run python -m boundflow_amd.build)")
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (bf_[a-z0-9_]+)$", out, flags=re.M))
    missing = [s for s in header_symbols() if s not in exported]
    assert not missing, missing
