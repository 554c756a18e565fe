"""Modulated deformable convolution (DCNv2) on MI355X (gfx950); same public names as
naotic/bev-kernels modulated_deform_conv/__init__.py."""
from .modulated_deform_conv import *  # noqa: F401,F403
from .modulated_deform_conv import (  # noqa: F401
    ModulatedDeformConv2dFunction,
    ModulatedDeformConv2d,
    ModulatedDeformConv2dPack,
    modulated_deform_conv2d,
    ext_modulated_deformable_col2im_opt,
    ext_modulated_deformable_col2im_smem,
    ext_modulated_deformable_col2im_coord_opt,
)
