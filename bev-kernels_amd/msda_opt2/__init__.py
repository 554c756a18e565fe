"""Multi-scale deformable attention on MI355X (gfx950)."""
from .dispatch import ms_deform_attn_backward, ms_deform_attn_forward
from .function import MultiScaleDeformableAttnFunction, multi_scale_deformable_attn

__all__ = [
    "ms_deform_attn_forward",
    "ms_deform_attn_backward",
    "MultiScaleDeformableAttnFunction",
    "multi_scale_deformable_attn",
]
