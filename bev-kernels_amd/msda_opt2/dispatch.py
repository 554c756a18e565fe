"""Multi-scale deformable attention entry points with the signatures of
naotic/bev-kernels msda_musa_opt2/msda_musa_opt2/dispatch.py:15-69, running on the
gfx950 kernels of libbevk.so (registered in ``_modulated_deform_conv_ext``)."""
from __future__ import annotations

from typing import Optional, Tuple

import torch


def _ext():
    import _modulated_deform_conv_ext
    return _modulated_deform_conv_ext


def ms_deform_attn_forward(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    level_start_index: torch.Tensor,
    sampling_loc: torch.Tensor,
    attn_weight: torch.Tensor,
    *,
    im2col_step: int = 64,
    force_generic: bool = False,
) -> torch.Tensor:
    """value [B, S, heads, D], spatial_shapes [L, 2] int64, level_start_index [L] int64,
    sampling_loc [B, Lq, heads, L, P, 2] in [0, 1], attn_weight [B, Lq, heads, L, P]
    -> [B, Lq, heads * D]. fp32 / fp16 / bf16 (fp32 accumulation) / fp64."""
    if not torch.cuda.is_available():
        raise RuntimeError("ms_deform_attn_forward requires a HIP device (torch.cuda)")
    return _ext().forward(value, spatial_shapes, level_start_index, sampling_loc, attn_weight,
                          im2col_step=im2col_step, force_generic=force_generic)


def ms_deform_attn_backward(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    level_start_index: torch.Tensor,
    sampling_loc: torch.Tensor,
    attn_weight: torch.Tensor,
    grad_output: torch.Tensor,
    *,
    im2col_step: int = 64,
    force_generic_col2im: bool = False,
    max_workspace_bytes: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients (value, sampling_loc, attn_weight) of ms_deform_attn_forward for
    grad_output [B, Lq, heads * D]. fp32 / fp64, and fp16 / bf16 with fp32 arithmetic and
    an fp32 grad_value accumulator. max_workspace_bytes (keyword only, not in the
    reference) caps the scratch: above it the atomic kernels run with the reference's
    memory use (default: the BEVK_MSDA_BACKWARD_MAX_WORKSPACE environment variable,
    unset = no cap)."""
    if not torch.cuda.is_available():
        raise RuntimeError("ms_deform_attn_backward requires a HIP device (torch.cuda)")
    grad_value = torch.zeros_like(value)
    grad_sampling_loc = torch.zeros_like(sampling_loc)
    grad_attn_weight = torch.zeros_like(attn_weight)
    _ext().backward(value, spatial_shapes, level_start_index, sampling_loc, attn_weight,
                    grad_output, grad_value, grad_sampling_loc, grad_attn_weight,
                    im2col_step=im2col_step, force_generic_col2im=force_generic_col2im,
                    max_workspace_bytes=max_workspace_bytes)
    return grad_value, grad_sampling_loc, grad_attn_weight
