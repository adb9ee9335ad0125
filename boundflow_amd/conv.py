"""Conv2d pieces of the HIP CROWN path (IBP conv and the conv backward step)."""

from __future__ import annotations


def ibp_conv2d(in_lo, in_hi, relu_in, layer, split, split_ld, lo, hi, infeasible):
    raise NotImplementedError("HIP conv2d IBP is not built yet")


def conv_backward_step(layer, is_first, A_u, A_l, stride, b_u, b_l, B, S, pre_lo, pre_hi, alpha, alpha_ld, add,
                       add_ld, spec, trace):
    raise NotImplementedError("HIP conv2d CROWN backward is not built yet")
