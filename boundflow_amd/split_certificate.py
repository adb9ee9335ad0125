"""First-layer split infeasibility certificate on the device.

Counterpart of ``_collect_first_layer_split_halfspaces`` and
``_is_infeasible_split_first_layer_convex_combo``
(boundflow/runtime/alpha_beta_crown.py:259-389, :391-532), which the
reference runs before a single-domain alpha-beta evaluation with splits
(:694-714), on every node of the per-node fallback of a node batch
(boundflow/runtime/bab.py:1399-1456) and as the optional pre-pruning of a
node batch (bab.py:373-425).

A split s on a ReLU whose input is produced from the network input by one
linear or conv2d op is the halfspace s * (r . x + b) >= 0, with r the
neuron's row of the weight (or of the conv's Jacobian).  ``bf_split_certificate``
searches, one workgroup per node, for a convex combination of a node's
halfspaces whose maximum over the input set is below -tol (the reference's
200-step softmax/Adam search), and flags the node infeasible when it finds
one.  The rows are read from the layer weight in place; a conv layer's
Jacobian rows are made once per weight tensor (kept across queries).
"""

from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch

from . import _lib
from .crown import derived
from .spec import BoxPerturbation, InputSpec, input_norm_p, normalize_input_spec


def _pair(v) -> Tuple[int, int]:
    if isinstance(v, int):
        return (v, v)
    v = tuple(int(x) for x in v)
    return (v[0], v[0]) if len(v) == 1 else (v[0], v[1])


# identity rows pulled back per launch when a conv's Jacobian is built (a 1024 x n_out block)
JACOBIAN_CHUNK = 1024


def _conv_jacobian(W: torch.Tensor, attrs, in_shape, out_shape) -> torch.Tensor:
    """Rows of the conv's Jacobian, [Co*Ho*Wo, Ci*Hi*Wi]: identity rows pulled back
    through the transposed convolution of the library, JACOBIAN_CHUNK rows at a
    time (the identity block of a chunk is the only temporary)."""
    Co, Ho, Wo = out_shape
    Ci, Hi, Wi = in_shape
    KH, KW = int(W.shape[2]), int(W.shape[3])
    sh, sw = _pair(attrs.get("stride", 1))
    ph, pw = _pair(attrs.get("padding", 0))
    n_out = Co * Ho * Wo
    rows = torch.empty(n_out, Ci * Hi * Wi, device=W.device, dtype=torch.float32)
    Wc = W.contiguous()
    stream = _lib.stream_handle()
    block = torch.empty(min(JACOBIAN_CHUNK, n_out), n_out, device=W.device, dtype=torch.float32)
    for r0 in range(0, n_out, JACOBIAN_CHUNK):
        m = min(JACOBIAN_CHUNK, n_out - r0)
        eye = block[:m]
        eye.zero_()
        eye.diagonal(offset=r0).fill_(1.0)
        _lib.call("bf_conv_transpose_rows", _lib.ptr(eye), None, m, Co, Ho, Wo, _lib.ptr(Wc), Ci, KH, KW,
                  sh, sw, ph, pw, Hi, Wi, _lib.ptr(rows[r0:r0 + m]), None, 1, None, 0, 0, None, None, None, None,
                  stream)
    return rows


def first_layer_sources(module, spec: InputSpec, relu_shapes: Dict[str, Tuple[int, ...]]):
    """[(relu input name, rows [n, I], bias [n] or None)] for every ReLU (op order)
    whose input is made by a linear or conv2d op reading the network input
    (the halfspace sources of alpha_beta_crown.py:259-389)."""
    task = module.get_entry_task()
    params = module.params
    producer = {op.outputs[0]: op for op in task.ops if op.outputs}
    in_shape = tuple(int(d) for d in spec.center.shape[1:])
    out: List[Tuple[str, torch.Tensor, Optional[torch.Tensor]]] = []
    for op in task.ops:
        if op.op_type != "relu":
            continue
        x = op.inputs[0]
        prod = producer.get(x)
        if prod is None or not prod.inputs or prod.inputs[0] != spec.value_name or x not in relu_shapes:
            continue
        W = params.get(prod.inputs[1])
        b = params.get(prod.inputs[2]) if len(prod.inputs) == 3 else None
        if prod.op_type == "linear" and len(prod.inputs) == 3 and b is None:
            continue   # a named bias missing from the parameters: the reference skips the layer (:306-308)
        n = 1
        for d in relu_shapes[x]:
            n *= int(d)
        if prod.op_type == "linear":
            if W is None or W.dim() != 2 or int(W.shape[0]) != n:
                continue
            if b is not None and (b.dim() != 1 or int(b.shape[0]) != n):
                continue
            out.append((x, W.contiguous(), None if b is None else b.contiguous()))
        elif prod.op_type == "conv2d":
            oshape = tuple(int(d) for d in relu_shapes[x])
            if W is None or W.dim() != 4 or len(in_shape) != 3 or len(oshape) != 3:
                continue
            a = prod.attrs
            if int(a.get("groups", 1)) != 1 or _pair(a.get("dilation", 1)) != (1, 1):
                raise NotImplementedError("first-layer split certificate: conv2d with groups or dilation != 1")
            rows = derived(f"conv_jacobian:{in_shape}:{oshape}:{a.get('stride', 1)}:{a.get('padding', 0)}", (W,),
                           lambda: _conv_jacobian(W, a, in_shape, oshape))
            bmap = None
            if b is not None:
                Co, Ho, Wo = oshape
                bmap = derived(f"conv_bias_map:{Ho}x{Wo}", (b,),
                               lambda: b.reshape(Co, 1).expand(Co, Ho * Wo).reshape(-1).contiguous())
            out.append((x, rows, bmap))
    return out


def split_certificate(module, input_spec, relu_split_state: Dict[str, torch.Tensor],
                      relu_shapes: Dict[str, Tuple[int, ...]], *, steps: int = 200, lr: float = 0.1,
                      tol: float = 1e-6, max_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """int32 [B] on the device: 1 where the first-layer splits of domain b (row b
    of each split tensor, or a shared row) are proven infeasible over domain b's
    input set, 0 otherwise (also when the domain has no first-layer split).
    ``max_out`` (optional, float32 [B] on the device) receives the smallest maximum of
    each domain's search (the certificate's value where the flag is 1).
    No host synchronization."""
    spec = normalize_input_spec(input_spec)
    B = int(spec.center.shape[0])
    dev = spec.center.device
    flags = torch.zeros(B, dtype=torch.int32, device=dev)
    sources = [s for s in first_layer_sources(module, spec, relu_shapes) if s[0] in (relu_split_state or {})]
    if max_out is not None:
        max_out.zero_()
    if not sources or B == 0:
        return flags
    I = int(spec.center[0].numel())
    pert = spec.perturbation
    if isinstance(pert, BoxPerturbation):
        lo = pert.lower.reshape(B, I)
        hi = pert.upper.reshape(B, I)
        center = ((lo + hi) / 2.0).contiguous()
        rad = ((hi - lo) / 2.0).contiguous()
        eps = 0.0
    else:
        center = spec.center.reshape(B, I).contiguous()
        rad = None
        eps = float(pert.eps)
    norm_p = input_norm_p(pert)

    def split_rows(name: str, n: int) -> torch.Tensor:
        s = relu_split_state[name].to(device=dev, dtype=torch.int8)
        if s.numel() == n:
            s = s.reshape(1, n).expand(B, n)
        return s.reshape(B, n)

    if len(sources) == 1:
        name, rows, bias = sources[0]
        n = int(rows.shape[0])
        split = split_rows(name, n)
        ld = 0 if split.stride(0) == 0 else n
        split = split if ld == 0 else split.contiguous()
    else:
        # several first layers: their halfspaces in op order, as one row set
        rows = torch.cat([r for _n, r, _b in sources], dim=0)
        if any(b is not None for _n, _r, b in sources):
            bias = torch.cat([b if b is not None else torch.zeros(int(r.shape[0]), device=dev)
                              for _n, r, b in sources])
        else:
            bias = None
        n = int(rows.shape[0])
        split = torch.cat([split_rows(nm, int(r.shape[0])) for nm, r, _b in sources], dim=1).contiguous()
        ld = n
    _lib.call("bf_split_certificate", _lib.ptr(rows), int(rows.stride(0)), _lib.ptr(bias), _lib.ptr(split), ld,
              _lib.ptr(center), I, _lib.ptr(rad), I if rad is not None else 0, float(eps), norm_p, B, n, I, int(steps),
              float(lr), float(tol), _lib.ptr(flags), _lib.ptr(max_out), _lib.stream_handle())
    return flags


def check_flags(flags_host: List[int]) -> None:
    """Raise when a node had more first-layer splits than the kernel's LDS stage holds."""
    if any(int(f) < 0 for f in flags_host):
        raise NotImplementedError("first-layer split certificate: more than 1024 first-layer splits on one node")
