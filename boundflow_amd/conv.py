"""Conv2d pieces of the HIP CROWN path.

* ``ibp_conv2d`` -- interval conv in center/radius form (``bf_ibp_conv2d``),
  the counterpart of the reference's W+/W- conv transformer
  (boundflow/domains/interval.py:57-74) after ``bounding_box`` for the input
  layer (boundflow/runtime/crown_ibp.py:167-181).
* ``conv_backward_step`` -- one ReLU -> Conv2d region of the CROWN backward.
  Inner layers: one pass (``bf_crown_relu_conv_transpose``) that relaxes each
  coefficient row while the transposed convolution stages it (the sign split of
  runtime/linear_operator.py:722-905 taken into the conv operator of
  :1067-1092), with the bias terms reduced in the same pass.  The input layer,
  and shapes that pass does not take: the relaxation pass
  (``bf_crown_relu_relax_lu``, with the conv bias map and, on the input layer, the
  center projection reduced in the same pass), then the transposed convolution
  (``bf_conv_transpose_rows``), fused with the Linf / box concretization on the
  input layer.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .profiling import launch as _timed
from .spec import BoxPerturbation, IntervalState, input_norm_p



def packed_conv_transpose_weights(W: torch.Tensor, Co: int, Ho: int, Wo: int, Ci: int, KH: int, KW: int, sh: int,
                                  sw: int, ph: int, pw: int, Hi: int, Wi: int, source=None) -> torch.Tensor:
    """The weights of the channel-last transposed convolution in its LDS order
    (bf_conv_transpose_pack_weights), made once per weight tensor and geometry and kept
    across queries (``source``: the tensor they derive from, default W)."""
    geo = (Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi)

    def pack():
        out = torch.empty(int(_lib.load().bf_conv_transpose_packed_floats(*geo)), device=W.device)
        _lib.call("bf_conv_transpose_pack_weights", _lib.ptr(W), *geo, _lib.ptr(out), _lib.stream_handle())
        return out
    return derived("conv_t_pack:" + "x".join(str(v) for v in geo), (W if source is None else source,), pack)

def _numel(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


def ibp_conv2d(in_lo, in_hi, relu_in, layer, split, split_ld, lo, hi, infeasible, *, linf_eps=None,
               center_out=None):
    Ci, Hi, Wi = layer.in_shape
    Co, Ho, Wo = layer.out_shape
    KH, KW = int(layer.weight.shape[2]), int(layer.weight.shape[3])
    sh, sw = layer.attrs["stride"]
    ph, pw = layer.attrs["padding"]
    B = int(in_lo.shape[0])
    ws = torch.empty(int(_lib.load().bf_ibp_conv2d_workspace(B, Ci * Hi * Wi, Co * Ho * Wo)), device=in_lo.device,
                     dtype=torch.float32)
    kind = 1 if linf_eps is not None else 0
    _lib.call("bf_ibp_conv2d", _lib.ptr(in_lo.contiguous()), _lib.ptr(None if in_hi is None else in_hi.contiguous()),
              B, Ci, Hi, Wi, kind, float(linf_eps or 0.0), int(relu_in), _lib.ptr(layer.weight.contiguous()),
              _lib.ptr(None if layer.bias is None else layer.bias.contiguous()), Co, KH, KW, sh, sw, ph, pw, Ho, Wo,
              _lib.ptr(split), split_ld, _lib.ptr(ws), _lib.ptr(lo), _lib.ptr(hi), _lib.ptr(center_out),
              _lib.ptr(infeasible), _lib.stream_handle())


def derived(tag, sources, make):
    from .crown import derived as _derived
    return _derived(tag, sources, make)


def call_memo(save, key, make):
    from .crown import call_memo as _call_memo
    return _call_memo(save, key, make)


def conv_backward_step(layer, is_first, A_u, A_l, stride, b_u, b_l, B, S, pre_lo, pre_hi, alpha, alpha_ld, add,
                       add_ld, spec, trace, save=None):
    """Returns (A_u, A_l, b_u, b_l, stride, done) where ``done`` is the final
    IntervalState on the input layer and None otherwise."""
    dev = spec.center.device
    stream = _lib.stream_handle()
    M = B * S
    Co, Ho, Wo = layer.out_shape
    Ci, Hi, Wi = layer.in_shape
    n_out = Co * Ho * Wo
    n_in = Ci * Hi * Wi
    KH, KW = int(layer.weight.shape[2]), int(layer.weight.shape[3])
    sh, sw = layer.attrs["stride"]
    ph, pw = layer.attrs["padding"]
    W = layer.weight.contiguous()

    def materialize(A):
        if A is None:
            return None
        if stride == S * n_out:
            return A.reshape(M, n_out)
        return A.reshape(-1, n_out)[: S].unsqueeze(0).expand(B, S, n_out).reshape(M, n_out).contiguous()

    A_u = materialize(A_u)
    A_l = materialize(A_l)
    kbias = None
    if layer.bias is not None:
        kbias = derived(f"conv_bias_map:{Ho}x{Wo}", (layer.bias,),
                        lambda: layer.bias.reshape(Co, 1).expand(Co, Ho * Wo).reshape(n_out).contiguous())
    cvec = trace.input_center_proj.get(layer.out_name) if is_first else None
    nz = int(A_u is not None) + int(A_l is not None)
    taps = KH * KW / float(sh * sw)
    flops = 2.0 * nz * M * n_in * Co * taps
    if not is_first and _lib.load().bf_conv_transpose_hwc_supported(Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi):
        # the relaxation applied while the transposed convolution stages each row: the relaxed
        # rows reach HBM only when the gradient pass needs them
        y_u = torch.empty(M, n_in, device=dev) if A_u is not None else None
        y_l = torch.empty(M, n_in, device=dev) if A_l is not None else None
        nb_u = torch.empty(M, device=dev) if A_u is not None else None
        nb_l = torch.empty(M, device=dev) if A_l is not None else None
        keep_l = torch.empty_like(A_l) if (save is not None and A_l is not None) else None
        packed = packed_conv_transpose_weights(W, Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi,
                                               source=layer.weight)
        with _timed("crown_relu_conv_transpose", flops,
                    4.0 * nz * (M * n_out + M * n_in) + (4.0 * M * n_out if keep_l is not None else 0.0)):
            _lib.call("bf_crown_relu_conv_transpose", _lib.ptr(A_u), _lib.ptr(A_l), B, S, Co, Ho, Wo, _lib.ptr(pre_lo),
                      _lib.ptr(pre_hi), _lib.ptr(alpha), alpha_ld, _lib.ptr(add), add_ld, _lib.ptr(kbias),
                      _lib.ptr(b_u), _lib.ptr(b_l), _lib.ptr(W), _lib.ptr(packed), Ci, KH, KW, sh, sw, ph, pw, Hi, Wi,
                      _lib.ptr(y_u), _lib.ptr(y_l), _lib.ptr(nb_u), _lib.ptr(nb_l), None, _lib.ptr(keep_l), stream)
        if save is not None:
            save.setdefault("relaxed", {})[layer.op_index] = keep_l
        return y_u, y_l, nb_u, nb_l, S * n_in, None
    nb_u = torch.empty(M, device=dev) if A_u is not None else None
    nb_l = torch.empty(M, device=dev) if A_l is not None else None
    c_u = torch.empty(M, device=dev) if (A_u is not None and cvec is not None) else None
    c_l = torch.empty(M, device=dev) if (A_l is not None and cvec is not None) else None
    if is_first and cvec is not None and _lib.load().bf_conv_transpose_small_supported(
            Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi):
        # input layer: relaxation, transposed conv and concretization norm in one pass
        return _input_layer_fused(spec, save, A_u, A_l, b_u, b_l, B, S, M, pre_lo, pre_hi, alpha, alpha_ld, add,
                                  add_ld, kbias, cvec, W, geo=(Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi),
                                  nb=(nb_u, nb_l), c=(c_u, c_l), flops=flops, nz=nz, layer=layer)
    rA_u = torch.empty_like(A_u) if A_u is not None else None
    rA_l = torch.empty_like(A_l) if A_l is not None else None
    with _timed("crown_relu_relax", 0.0, 4.0 * nz * 2 * M * n_out):
        _lib.call("bf_crown_relu_relax_lu", _lib.ptr(A_u), _lib.ptr(A_l), S * n_out, B, S, n_out, _lib.ptr(pre_lo),
                  _lib.ptr(pre_hi), _lib.ptr(alpha), alpha_ld, _lib.ptr(add), add_ld, _lib.ptr(kbias), _lib.ptr(cvec),
                  _lib.ptr(b_u), _lib.ptr(b_l), _lib.ptr(rA_u), _lib.ptr(rA_l), _lib.ptr(nb_u), _lib.ptr(nb_l),
                  _lib.ptr(c_u), _lib.ptr(c_l), stream)
    if not is_first:
        y_u = torch.empty(M, n_in, device=dev) if A_u is not None else None
        y_l = torch.empty(M, n_in, device=dev) if A_l is not None else None
        with _timed("conv_transpose", flops, 4.0 * nz * (M * n_out + M * n_in)):
            _lib.call("bf_conv_transpose_rows", _lib.ptr(rA_u), _lib.ptr(rA_l), M, Co, Ho, Wo, _lib.ptr(W), Ci, KH,
                      KW, sh, sw, ph, pw, Hi, Wi, _lib.ptr(y_u), _lib.ptr(y_l), S, None, 0, 0, None, None, None,
                      None, stream)
        if save is not None:
            save.setdefault("relaxed", {})[layer.op_index] = rA_l
        return y_u, y_l, nb_u, nb_l, S * n_in, None
    # input layer: transposed conv fused with the concretization
    pert = spec.perturbation
    norm_p = input_norm_p(pert)
    if cvec is None:
        raise RuntimeError("forward trace lacks the input-layer projection")
    if isinstance(pert, BoxPerturbation):
        rad = ((pert.upper - pert.lower) / 2.0).reshape(B, n_in).contiguous()
        eps = 1.0
    else:
        rad = None
        eps = float(pert.eps)
    norm_u = torch.empty(M, device=dev) if A_u is not None else None
    norm_l = torch.empty(M, device=dev) if A_l is not None else None
    h_scale = h_out = None
    if save is not None and save.get("grad_rows") is not None:
        h_scale = call_memo(save, f"h_scale:{eps!r}", lambda: (save["grad_rows"] * (-eps)).contiguous())
        h_out = torch.empty(M, n_in, device=dev)
        save["h"] = h_out
        save["cvec"] = cvec
    with _timed("conv_transpose_concretize", flops, 4.0 * nz * M * n_out):
        _lib.call("bf_conv_transpose_rows", _lib.ptr(rA_u), _lib.ptr(rA_l), M, Co, Ho, Wo, _lib.ptr(W), Ci, KH, KW,
                  sh, sw, ph, pw, Hi, Wi, None, None, S, _lib.ptr(rad), n_in, norm_p, _lib.ptr(norm_u),
                  _lib.ptr(norm_l), _lib.ptr(h_scale), _lib.ptr(h_out), stream)
    if save is not None:
        save.setdefault("relaxed", {})[layer.op_index] = rA_l
    lb = torch.empty(B, S, device=dev) if A_l is not None else None
    ub = torch.empty(B, S, device=dev) if A_u is not None else None
    _lib.call("bf_concretize_finalize", _lib.ptr(norm_u), _lib.ptr(norm_l), 1, M, _lib.ptr(c_u), _lib.ptr(c_l),
              _lib.ptr(nb_u), _lib.ptr(nb_l), eps, norm_p, _lib.ptr(lb), _lib.ptr(ub), stream)
    return None, None, None, None, 0, IntervalState(lower=lb, upper=ub)


def _input_layer_fused(spec, save, A_u, A_l, b_u, b_l, B, S, M, pre_lo, pre_hi, alpha, alpha_ld, add, add_ld, kbias,
                       cvec, W, geo, nb, c, flops, nz, layer):
    """The input conv layer through bf_crown_relu_conv_transpose_concretize: the ReLU
    relaxation applied while each row is staged, the transposed conv reduced to the
    concretization norm (and the gradient seed), the relaxed rows written only for a
    gradient pass; the bounds from the norms, centers and biases in the same launch."""
    dev = spec.center.device
    stream = _lib.stream_handle()
    norm_p = input_norm_p(spec.perturbation)
    Co, Ho, Wo, Ci, KH, KW, sh, sw, ph, pw, Hi, Wi = geo
    n_out, n_in = Co * Ho * Wo, Ci * Hi * Wi
    nb_u, nb_l = nb
    c_u, c_l = c
    pert = spec.perturbation
    if isinstance(pert, BoxPerturbation):
        rad = ((pert.upper - pert.lower) / 2.0).reshape(B, n_in).contiguous()
        eps = 1.0
    else:
        rad = None
        eps = float(pert.eps)
    norm_u = torch.empty(M, device=dev) if A_u is not None else None
    norm_l = torch.empty(M, device=dev) if A_l is not None else None
    h_scale = h_out = None
    if save is not None and save.get("grad_rows") is not None:
        h_scale = call_memo(save, f"h_scale:{eps!r}", lambda: (save["grad_rows"] * (-eps)).contiguous())
        h_out = torch.empty(M, n_in, device=dev)
        save["h"] = h_out
        save["cvec"] = cvec
    rel_l = torch.empty(M, n_out, device=dev) if (save is not None and A_l is not None) else None
    lb = torch.empty(B, S, device=dev) if A_l is not None else None
    ub = torch.empty(B, S, device=dev) if A_u is not None else None
    with _timed("crown_relu_conv_transpose_concretize", flops,
                4.0 * nz * (M * n_out + 2 * B * n_out) + (4.0 * M * n_out if rel_l is not None else 0.0)):
        _lib.call("bf_crown_relu_conv_transpose_concretize", _lib.ptr(A_u), _lib.ptr(A_l), B, S, Co, Ho, Wo,
                  _lib.ptr(pre_lo), _lib.ptr(pre_hi), _lib.ptr(alpha), alpha_ld, _lib.ptr(add), add_ld,
                  _lib.ptr(kbias), _lib.ptr(cvec), _lib.ptr(b_u), _lib.ptr(b_l), _lib.ptr(W), Ci, KH, KW, sh, sw, ph,
                  pw, Hi, Wi, _lib.ptr(rad), n_in, norm_p, _lib.ptr(h_scale), _lib.ptr(h_out), _lib.ptr(norm_u),
                  _lib.ptr(norm_l), _lib.ptr(nb_u), _lib.ptr(nb_l), _lib.ptr(c_u), _lib.ptr(c_l), None,
                  _lib.ptr(rel_l), eps, _lib.ptr(lb), _lib.ptr(ub), stream)
    if save is not None:
        save.setdefault("relaxed", {})[layer.op_index] = rel_l
    # the launch wrote the bounds (c -/+ eps * norm) + b of every row
    return None, None, None, None, 0, IntervalState(lower=lb, upper=ub)

