"""Autograd wrapper of the MSDA kernels in the form callers of mmcv's
``MultiScaleDeformableAttnFunction`` use (apply(value, spatial_shapes, level_start_index,
sampling_locations, attention_weights, im2col_step)). The reference exposes only the two
functions of dispatch.py:15-69 and leaves the Function to its callers."""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from .dispatch import ms_deform_attn_backward, ms_deform_attn_forward


class MultiScaleDeformableAttnFunction(torch.autograd.Function):
    """out [B, Lq, heads*D] = MSDA(value [B, S, heads, D], ...). Gradients flow to value,
    sampling_locations and attention_weights; spatial_shapes, level_start_index and
    im2col_step get none."""

    @staticmethod
    def forward(ctx, value, value_spatial_shapes, value_level_start_index,
                sampling_locations, attention_weights, im2col_step=64):
        ctx.im2col_step = im2col_step
        out = ms_deform_attn_forward(value, value_spatial_shapes, value_level_start_index,
                                     sampling_locations, attention_weights,
                                     im2col_step=im2col_step)
        ctx.save_for_backward(value, value_spatial_shapes, value_level_start_index,
                              sampling_locations, attention_weights)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        value, shapes, lsi, loc, attn = ctx.saved_tensors
        # the kernels read grad_output through its strides when it can be viewed as
        # [B, Lq, heads, D]; anything else (an expanded gradient) is made dense first
        B, _, NH, D = value.shape
        try:
            grad_output.view(B, loc.shape[1], NH, D)
        except RuntimeError:
            grad_output = grad_output.contiguous()
        g_value, g_loc, g_attn = ms_deform_attn_backward(
            value, shapes, lsi, loc, attn, grad_output, im2col_step=ctx.im2col_step)
        return g_value, None, None, g_loc, g_attn, None


def multi_scale_deformable_attn(value, spatial_shapes, level_start_index, sampling_locations,
                                attention_weights, im2col_step=64):
    """Differentiable MSDA: MultiScaleDeformableAttnFunction.apply."""
    return MultiScaleDeformableAttnFunction.apply(value, spatial_shapes, level_start_index,
                                                  sampling_locations, attention_weights,
                                                  im2col_step)
