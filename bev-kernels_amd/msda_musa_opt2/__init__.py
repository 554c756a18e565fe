"""Alias of ``msda_opt2`` under the reference's package name (msda_musa_opt2)."""
from msda_opt2 import ms_deform_attn_backward, ms_deform_attn_forward  # noqa: F401
from msda_opt2 import MultiScaleDeformableAttnFunction, multi_scale_deformable_attn  # noqa: F401
from msda_opt2 import dispatch  # noqa: F401

__all__ = [
    "ms_deform_attn_forward",
    "ms_deform_attn_backward",
    "MultiScaleDeformableAttnFunction",
    "multi_scale_deformable_attn",
]
