"""Packed main weight for the fused NHWC kernel.

The fused kernel reads the weight in the layout dcn_pack_weight produces (MFMA-fragment
blocks for fp16 / bf16, [Cout][kh][kw][C] for fp32). The weight is packed on every call,
as the reference flattens its weight on every call (dcn_split_nhwc.py:143,
fused_tl.py:399): one small kernel (a few microseconds for a 256 x 256 x 3 x 3 weight)
beside the convolution, and no cached copy that a write through ``weight.data``, an EMA
swap or another kernel could leave stale.
"""
from __future__ import annotations

import torch


def _ext():
    import _modulated_deform_conv_ext as ext
    return ext


def pack_weight(weight: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Pack weight [Cout, C, kh, kw] converted to `dtype`."""
    return _ext().dcn_pack_weight(weight.detach().to(dtype).contiguous())
