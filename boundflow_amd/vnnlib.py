"""VNNLIB box properties: parse a property file into a query of an input box and
an OR of linear unsafe clauses, and turn it into the tensors the bound runtime
takes (a box input spec, a spec matrix C and thresholds).

Counterpart of boundflow/frontends/vnnlib.py (``parse_vnnlib_box_query``,
``import_vnnlib_box_query``, ``materialize_vnnlib_box_query``) and of the query
IR of boundflow/ir/query.py (``LinearUnsafeClauseIR``, ``VNNLibBoxQueryIR``).
The accepted subset is the reference's, and like it the parser fails closed
(ValueError) on anything else:

* ``(declare-const X_i Real)`` / ``(declare-const Y_j Real)``, each once;
* one lower and one upper scalar bound per input, ``(<= X_i c)``, ``(>= c X_i)``
  and the mirrored forms;
* exactly one output assertion ``(or d_0 d_1 ...)``; each disjunct is one linear
  relation (optionally wrapped in a one-argument ``and``) between linear
  expressions of the outputs built from ``+``, ``-``, scalar ``*`` and constants.

A disjunct ``lhs >= rhs`` (or ``>``) becomes the margin m = rhs - lhs, and
``lhs <= rhs`` (``<``) m = lhs - rhs; the property is unsafe when some margin
satisfies c . y <= threshold, with c the margin's coefficients on the outputs and
threshold = -(its constant).  Verifying the property means a lower bound of
every c . y above its threshold.
"""

from __future__ import annotations

import hashlib
import json
import math
import re
from dataclasses import dataclass
from pathlib import Path
from typing import List, Sequence, Tuple, Union

import torch

VNNLIB_BOX_QUERY_IR_SCHEMA_VERSION = "boundflow.vnnlib_box_query_ir/v1"

SExpr = Union[str, list]
_VAR = re.compile(r"([XY])_(0|[1-9][0-9]*)\Z")


def _is_sha256(v: object) -> bool:
    return isinstance(v, str) and len(v) == 64 and all(ch in "0123456789abcdef" for ch in v)


def _canonical_hash(value: object) -> str:
    text = json.dumps(value, sort_keys=True, separators=(",", ":"), allow_nan=False)
    return hashlib.sha256(text.encode("utf-8")).hexdigest()


@dataclass(frozen=True)
class LinearUnsafeClauseIR:
    """One unsafe disjunct as a margin c . y with the threshold it must not exceed."""

    ordinal: int
    coefficients: Tuple[float, ...]
    threshold: float
    source_relation: str
    source_expression_hash: str

    def validate(self) -> None:
        ok = (self.ordinal >= 0 and len(self.coefficients) > 0
              and all(math.isfinite(c) for c in self.coefficients)
              and any(c != 0.0 for c in self.coefficients)
              and math.isfinite(self.threshold)
              and self.source_relation in (">=", ">", "<=", "<")
              and _is_sha256(self.source_expression_hash))
        if not ok:
            raise ValueError("linear unsafe clause IR is invalid")

    def to_dict(self) -> dict:
        self.validate()
        return {"ordinal": self.ordinal, "coefficients": list(self.coefficients), "threshold": self.threshold,
                "source_relation": self.source_relation, "source_expression_hash": self.source_expression_hash,
                "margin_semantics": "unsafe_when_margin_le_threshold"}

    def stable_hash(self) -> str:
        return _canonical_hash(self.to_dict())


@dataclass(frozen=True)
class VNNLibBoxQueryIR:
    """A bounded input box and an OR of single linear unsafe clauses."""

    query_id: str
    source_sha256: str
    input_names: Tuple[str, ...]
    output_names: Tuple[str, ...]
    input_lower: Tuple[float, ...]
    input_upper: Tuple[float, ...]
    unsafe_clauses: Tuple[LinearUnsafeClauseIR, ...]
    schema_version: str = VNNLIB_BOX_QUERY_IR_SCHEMA_VERSION

    def validate(self) -> None:
        n_in, n_out = len(self.input_names), len(self.output_names)
        ok = (self.schema_version == VNNLIB_BOX_QUERY_IR_SCHEMA_VERSION and bool(self.query_id)
              and _is_sha256(self.source_sha256)
              and self.input_names == tuple(f"X_{i}" for i in range(n_in))
              and self.output_names == tuple(f"Y_{j}" for j in range(n_out))
              and n_in > 0 and n_out > 0
              and len(self.input_lower) == n_in and len(self.input_upper) == n_in
              and len(self.unsafe_clauses) > 0
              and {len(c.coefficients) for c in self.unsafe_clauses} == {n_out}
              and all(math.isfinite(v) for v in self.input_lower + self.input_upper)
              and all(lo <= hi for lo, hi in zip(self.input_lower, self.input_upper)))
        if not ok:
            raise ValueError("VNNLIB box Query IR is invalid")
        for i, clause in enumerate(self.unsafe_clauses):
            clause.validate()
            if clause.ordinal != i:
                raise ValueError("VNNLIB unsafe clause ordinal differs")

    def to_dict(self) -> dict:
        self.validate()
        return {"schema_version": self.schema_version, "query_id": self.query_id,
                "source_sha256": self.source_sha256, "input_names": list(self.input_names),
                "output_names": list(self.output_names), "input_lower": list(self.input_lower),
                "input_upper": list(self.input_upper),
                "unsafe_clauses": [c.to_dict() for c in self.unsafe_clauses],
                "property_aggregation": "all_unsafe_disjuncts_must_be_refuted", "performance_claimed": False}

    def stable_hash(self) -> str:
        return _canonical_hash(self.to_dict())


# ---------------------------------------------------------------------------
# S-expressions


def _read(text: str) -> List[SExpr]:
    """Top-level s-expressions of ``text`` (``;`` comments to end of line)."""
    body = "\n".join(line.split(";", 1)[0] for line in text.splitlines())
    tokens = re.findall(r"\(|\)|[^\s()]+", body)
    stack: List[list] = [[]]
    for tok in tokens:
        if tok == "(":
            stack.append([])
        elif tok == ")":
            if len(stack) == 1:
                raise ValueError("VNNLIB contains an unmatched closing parenthesis")
            done = stack.pop()
            stack[-1].append(done)
        else:
            stack[-1].append(tok)
    if len(stack) != 1:
        raise ValueError("VNNLIB contains an unmatched opening parenthesis")
    if not stack[0]:
        raise ValueError("VNNLIB source is empty")
    return stack[0]


def _encode(e: SExpr) -> str:
    return e if isinstance(e, str) else "(" + " ".join(_encode(x) for x in e) + ")"


def _as_list(e: SExpr, what: str) -> list:
    if not isinstance(e, list) or not e:
        raise ValueError(f"{what} must be a non-empty expression")
    return e


def _as_atom(e: SExpr, what: str) -> str:
    if not isinstance(e, str):
        raise ValueError(f"{what} must be an atom")
    return e


def _as_number(e: SExpr, what: str) -> float:
    try:
        v = float(_as_atom(e, what))
    except ValueError as err:
        raise ValueError(f"{what} must be numeric") from err
    if not math.isfinite(v):
        raise ValueError(f"{what} must be finite")
    return v


def _names(e: SExpr) -> set:
    if isinstance(e, str):
        return {e} if _VAR.fullmatch(e) else set()
    return set().union(*(_names(x) for x in e)) if e else set()


def _index(name: str, prefix: str) -> int:
    m = _VAR.fullmatch(name)
    if m is None or m.group(1) != prefix:
        raise ValueError(f"expected a {prefix} variable, got {name!r}")
    return int(m.group(2))


# ---------------------------------------------------------------------------
# Input bounds and output clauses


def _input_bound(e: SExpr) -> Tuple[str, str, float]:
    """(variable, "lower"|"upper", value) of one scalar input bound."""
    rel = _as_list(e, "VNNLIB input assertion")
    if len(rel) != 3 or _as_atom(rel[0], "input relation") not in ("<=", ">="):
        raise ValueError("VNNLIB input assertion must be one scalar <=/>= bound")
    op = rel[0]
    a = _as_atom(rel[1], "input bound left operand")
    b = _as_atom(rel[2], "input bound right operand")
    a_var = bool(_VAR.fullmatch(a)) and a.startswith("X_")
    b_var = bool(_VAR.fullmatch(b)) and b.startswith("X_")
    if a_var == b_var:
        raise ValueError("VNNLIB input bound must compare one X variable and one scalar")
    if a_var:   # X op c
        return a, ("upper" if op == "<=" else "lower"), _as_number(b, "input bound scalar")
    return b, ("lower" if op == "<=" else "upper"), _as_number(a, "input bound scalar")   # c op X


def _affine(e: SExpr, n_out: int) -> Tuple[List[float], float]:
    """(coefficients on Y, constant) of a linear output expression."""
    if isinstance(e, str):
        m = _VAR.fullmatch(e)
        if m is None:
            return [0.0] * n_out, _as_number(e, "linear constant")
        if m.group(1) != "Y":
            raise ValueError("VNNLIB output constraint cannot reference X variables")
        j = int(m.group(2))
        if j >= n_out:
            raise ValueError("VNNLIB output variable index is out of range")
        coef = [0.0] * n_out
        coef[j] = 1.0
        return coef, 0.0
    items = _as_list(e, "linear output expression")
    op = _as_atom(items[0], "linear output operator")
    args = [_affine(a, n_out) for a in items[1:]]

    def add(x, y, sy=1.0):
        return [p + sy * q for p, q in zip(x[0], y[0])], x[1] + sy * y[1]

    def scale(x, s):
        return [s * p for p in x[0]], s * x[1]

    if op == "+" and args:
        acc = ([0.0] * n_out, 0.0)
        for a in args:
            acc = add(acc, a)
        return acc
    if op == "-" and args:
        if len(args) == 1:
            return scale(args[0], -1.0)
        acc = args[0]
        for a in args[1:]:
            acc = add(acc, scale(a, -1.0))
        return acc
    if op == "*" and len(args) == 2:
        l_const = not any(args[0][0])
        r_const = not any(args[1][0])
        if l_const == r_const:
            raise ValueError("VNNLIB multiplication must contain one scalar factor")
        return scale(args[1], args[0][1]) if l_const else scale(args[0], args[1][1])
    raise ValueError(f"unsupported VNNLIB linear operator: {op!r}")


def _clause(e: SExpr, *, ordinal: int, n_out: int) -> LinearUnsafeClauseIR:
    branch = _as_list(e, "VNNLIB unsafe disjunct")
    if _as_atom(branch[0], "unsafe disjunct operator") == "and":
        if len(branch) != 2:
            raise ValueError("VNNLIB v1 requires one inequality per unsafe disjunct")
        branch = _as_list(branch[1], "VNNLIB unsafe relation")
    if len(branch) != 3:
        raise ValueError("VNNLIB unsafe clause must be one binary relation")
    rel = _as_atom(branch[0], "VNNLIB unsafe relation")
    if rel not in (">=", ">", "<=", "<"):
        raise ValueError("VNNLIB unsafe relation is unsupported")
    lhs = _affine(branch[1], n_out)
    rhs = _affine(branch[2], n_out)
    # margin = (smaller side) - (larger side) of the unsafe relation
    small, large = (rhs, lhs) if rel in (">=", ">") else (lhs, rhs)
    coef = tuple(p - q for p, q in zip(small[0], large[0]))
    const = small[1] - large[1]
    clause = LinearUnsafeClauseIR(ordinal=ordinal, coefficients=coef, threshold=-const, source_relation=rel,
                                  source_expression_hash=hashlib.sha256(_encode(branch).encode("utf-8")).hexdigest())
    clause.validate()
    return clause


def parse_vnnlib_box_query(text: str, *, query_id: str, expected_source_sha256: str = None) -> VNNLibBoxQueryIR:
    """Parse the supported VNNLIB subset (module docstring) into the query IR."""
    digest = hashlib.sha256(text.encode("utf-8")).hexdigest()
    if expected_source_sha256 is not None and expected_source_sha256 != digest:
        raise ValueError("VNNLIB source digest differs")
    declared = {}
    in_asserts: List[SExpr] = []
    out_asserts: List[SExpr] = []
    for form in _read(text):
        form = _as_list(form, "VNNLIB top-level form")
        head = _as_atom(form[0], "VNNLIB top-level operator")
        if head == "declare-const":
            if len(form) != 3 or _as_atom(form[2], "declaration type") != "Real":
                raise ValueError("VNNLIB declaration must be a Real constant")
            name = _as_atom(form[1], "declaration name")
            if _VAR.fullmatch(name) is None or name in declared:
                raise ValueError("VNNLIB variable declaration is invalid or duplicated")
            declared[name] = "Real"
            continue
        if head != "assert" or len(form) != 2:
            raise ValueError(f"unsupported VNNLIB top-level form: {head!r}")
        used = _names(form[1])
        if not used or any(n not in declared for n in used):
            raise ValueError("VNNLIB assertion references missing/no variables")
        if all(n.startswith("X_") for n in used):
            in_asserts.append(form[1])
        elif all(n.startswith("Y_") for n in used):
            out_asserts.append(form[1])
        else:
            raise ValueError("VNNLIB assertion cannot mix input and output variables")
    xs = tuple(sorted((n for n in declared if n.startswith("X_")), key=lambda n: _index(n, "X")))
    ys = tuple(sorted((n for n in declared if n.startswith("Y_")), key=lambda n: _index(n, "Y")))
    bounds = {"lower": {}, "upper": {}}
    for a in in_asserts:
        name, side, value = _input_bound(a)
        if name in bounds[side]:
            raise ValueError(f"VNNLIB duplicates the {side} bound for {name}")
        bounds[side][name] = value
    if set(bounds["lower"]) != set(xs) or set(bounds["upper"]) != set(xs):
        raise ValueError("VNNLIB input box is incomplete")
    if len(out_asserts) != 1:
        raise ValueError("VNNLIB v1 requires exactly one output assertion")
    formula = _as_list(out_asserts[0], "VNNLIB output assertion")
    if _as_atom(formula[0], "VNNLIB output formula") != "or" or len(formula) < 2:
        raise ValueError("VNNLIB v1 output assertion must be a non-empty OR")
    clauses = tuple(_clause(b, ordinal=i, n_out=len(ys)) for i, b in enumerate(formula[1:]))
    query = VNNLibBoxQueryIR(query_id=query_id, source_sha256=digest, input_names=xs, output_names=ys,
                             input_lower=tuple(bounds["lower"][n] for n in xs),
                             input_upper=tuple(bounds["upper"][n] for n in xs), unsafe_clauses=clauses)
    query.validate()
    return query


def import_vnnlib_box_query(path: Union[str, Path], *, query_id: str) -> VNNLibBoxQueryIR:
    return parse_vnnlib_box_query(Path(path).read_text(encoding="utf-8"), query_id=query_id)


@dataclass(frozen=True)
class VNNLibQueryTensors:
    """The query as tensors: the input box [1, *shape], C [1, clauses, outputs], thresholds [clauses]."""

    input_lower: torch.Tensor
    input_upper: torch.Tensor
    linear_spec_c: torch.Tensor
    thresholds: torch.Tensor


def materialize_vnnlib_box_query(query: VNNLibBoxQueryIR, *, input_shape: Sequence[int],
                                 dtype: torch.dtype = torch.float32, device="cpu") -> VNNLibQueryTensors:
    query.validate()
    shape = tuple(int(d) for d in input_shape)
    if not shape or any(d < 1 for d in shape) or math.prod(shape) != len(query.input_names) \
            or not dtype.is_floating_point:
        raise ValueError("VNNLIB query tensor materialization shape/dtype differs")
    lo = torch.tensor(query.input_lower, dtype=dtype, device=device).reshape((1,) + shape)
    hi = torch.tensor(query.input_upper, dtype=dtype, device=device).reshape((1,) + shape)
    C = torch.tensor([c.coefficients for c in query.unsafe_clauses], dtype=dtype, device=device).unsqueeze(0)
    thr = torch.tensor([c.threshold for c in query.unsafe_clauses], dtype=dtype, device=device)
    return VNNLibQueryTensors(input_lower=lo, input_upper=hi, linear_spec_c=C, thresholds=thr)


def query_verified(lower: torch.Tensor, thresholds: torch.Tensor) -> bool:
    """A box property holds when every unsafe clause's margin lower bound exceeds its
    threshold (``unsafe_when_margin_le_threshold``); ``lower`` [1, clauses]."""
    return bool((lower.reshape(-1).to(thresholds.device, thresholds.dtype) > thresholds).all())
