"""Packed main weight for the fused NHWC kernel, cached on the weight tensor.

The fused kernel reads the weight in the layout dcn_pack_weight produces (MFMA-fragment
blocks for fp16 / bf16). A module's weight changes rarely, so the packed copy is kept on
the weight tensor itself and rebuilt when the tensor's storage, version counter (bumped
by every in-place update, optimizer steps included), dtype or device differs from the
one it was packed from.
"""
from __future__ import annotations

import torch

_ATTR = "_bevk_packed_weight"


def _ext():
    import _modulated_deform_conv_ext as ext
    return ext


def pack_weight(weight: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Pack weight [Cout, C, kh, kw] converted to `dtype` (no caching)."""
    return _ext().dcn_pack_weight(weight.detach().to(dtype).contiguous())


def packed_weight(weight: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Packed copy of weight [Cout, C, kh, kw] in `dtype`, reused while the weight is
    unchanged."""
    key = (weight.data_ptr(), weight._version, dtype, tuple(weight.shape), weight.device)
    hit = getattr(weight, _ATTR, None)
    if hit is not None and hit[0] == key:
        return hit[1]
    packed = pack_weight(weight, dtype)
    try:
        setattr(weight, _ATTR, (key, packed))
    except (AttributeError, RuntimeError):
        pass
    return packed
