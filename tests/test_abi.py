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


def header_declarations():
    """name -> (return type, [parameter types]) of every declaration in the header,
    each C type reduced to its ctypes class (pointers and hipStream_t are pointers)."""
    import ctypes
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    decls = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(bf_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()

        def ctype(decl: str):
            decl = " ".join(decl.split())
            if "*" in decl:
                return ctypes.c_void_p
            base = decl.replace("const ", "").split()
            if "hipStream_t" in base:
                return ctypes.c_void_p
            for key, ct in (("int64_t", ctypes.c_int64), ("int32_t", ctypes.c_int32), ("int", ctypes.c_int),
                            ("float", ctypes.c_float), ("double", ctypes.c_double)):
                if key in base:
                    return ct
            raise AssertionError(f"{name}: unknown C type {decl!r}")

        args = [] if params in ("", "void") else [ctype(p) for p in params.split(",")]
        r = ctypes.c_char_p if ret.replace(" ", "") == "constchar*" else ctype(ret)
        decls[name] = (r, args)
    return decls


def test_binding_argument_types_match_header():
    """Every parameter's C type (int / int64_t / float / double / pointer) equals the
    ctypes type the binding passes: a c_int for an int64_t stack argument would
    otherwise pass silently."""
    import ctypes
    from boundflow_amd import _lib
    decls = header_declarations()
    assert sorted(decls) == sorted(_lib.SIGNATURES)
    norm = {ctypes.c_int32: ctypes.c_int}
    for name, (res, args) in _lib.SIGNATURES.items():
        h_res, h_args = decls[name]
        assert norm.get(h_res, h_res) == norm.get(res, res), f"{name}: return type"
        assert len(h_args) == len(args), f"{name}: {len(h_args)} parameters in the header, {len(args)} bound"
        for i, (h, b) in enumerate(zip(h_args, args)):
            assert norm.get(h, h) == norm.get(b, b), f"{name}: parameter {i} is {h.__name__} in the header, " \
                                                     f"{b.__name__} in the binding"


def test_tile_configuration_rule():
    """The contraction's tile choice (a host-side rule, no device call): 128 x 128
    TileG for evenly loaded grids (C2), for grids of fewer 128 x 128 tiles than CUs the
    64 x 64 TileS with the plain prologue and TileH with the relaxation prologue (C1,
    C3, C4, D1), the 64 x 128 TileQ for C5's unevenly loaded 36 864-row grids
    on direct-to-LDS operands with the plain prologue, and 0 for bad sizes."""
    from boundflow_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built (run python -m boundflow_amd.build)")
    if os.environ.get("BOUNDFLOW_GEMM_TILE"):
        pytest.skip("tile forced by the environment")
    cfg = lambda *a: chr(_lib.load().bf_gemm_tile_config(*a)) if _lib.load().bf_gemm_tile_config(*a) else ""
    assert cfg(36864, 256, 1, 1, 0, 1) == "Q"      # C5 gradient / relaxation-epilogue contractions
    assert cfg(36864, 784, 1, 1, 0, 1) == "G"      # C5 concretization: 2016 tiles, even enough
    assert cfg(36864, 256, 2, 1, 0, 1) == "G"      # both bounds: 1152 tiles, 4.5 per CU either way
    assert cfg(128000, 500, 2, 1, 0, 1) == "G"     # C2 refinements
    assert cfg(2304, 500, 2, 1, 0, 1) == "S"       # a small grid, plain prologue
    assert cfg(2304, 500, 2, 1, 1, 1) == "H"       # C2's final spec query (relaxation prologue)
    assert cfg(36864, 256, 1, 1, 1, 1) == "G"      # relaxation prologue: TileQ takes the plain one only
    assert cfg(36864, 256, 1, 1, 0, 0) == "G"      # operands the direct-to-LDS loop does not take
    assert cfg(0, 256, 1, 1, 0, 1) == "" and cfg(10, 10, 3, 1, 0, 1) == ""
