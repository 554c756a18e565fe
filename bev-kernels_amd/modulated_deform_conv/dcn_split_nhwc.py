"""NHWC DCNv2: offset conv + deformable gather/GEMM, with the public names of
naotic/bev-kernels modulated_deform_conv/dcn_split_nhwc.py.

Layout: x [B,H,W,Cin], w_off [3T,Cin,kH,kW], b_off [3T], weight [Cout,Cin,kH,kW];
output [B,Ho,Wo,Cout].

The forward keeps the offset conv as a library convolution and runs the deformable
part as one gfx950 kernel that reads the raw offset-conv output y [B,Ho,Wo,3T] (offsets,
then the pre-sigmoid mask), builds the column tiles in LDS and multiplies them on the
matrix cores: the [M, T*Cin] column matrix never exists in HBM. ``gather_cols_nhwc``
still materialises it for callers that want the columns.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from ._packing import pack_weight, packed_weight


def out_size(H, pad, dil, k, stride):
    return (H + 2 * pad - (dil * (k - 1) + 1)) // stride + 1


def _ext():
    import _modulated_deform_conv_ext as ext
    return ext


def gather_cols_nhwc(x_nhwc, offset, mask=None, kH=3, kW=3, stride=1, padding=1, dilation=1):
    """Deformable gather -> columns [M, T*Cin], k = t*Cin + ci.

    Pass the raw offset-conv output y [B,Ho,Wo,3T] as ``offset`` with mask=None to read
    offsets from y[..., :2T] and mask = sigmoid(y[..., 2T:]); otherwise pass offset
    [B,Ho,Wo,2T] and mask [B,Ho,Wo,T]."""
    B, H, W, Cin = x_nhwc.shape
    Tt = kH * kW
    Ho = out_size(H, padding, dilation, kH, stride)
    Wo = out_size(W, padding, dilation, kW, stride)
    M = B * Ho * Wo
    off_c = offset.contiguous()
    mask_c = (mask if mask is not None else offset).contiguous()
    col = torch.empty(M, Tt * Cin, device=x_nhwc.device, dtype=x_nhwc.dtype)  # fully written
    _ext().modulated_deformable_im2col_nhwc_cuda(
        x_nhwc.contiguous(), off_c, mask_c, B, Cin, H, W, Ho, Wo, kH, kW, padding, padding,
        stride, stride, dilation, dilation, 1, col)
    return col


def col2im_nhwc(dcol, x_nhwc, offset, mask=None, kH=3, kW=3, stride=1, padding=1, dilation=1):
    """Backward col2im of the reference; the backward kernels are not part of this build."""
    raise RuntimeError("col2im_nhwc: the backward kernels are not part of this build "
                       "(forward operators only)")


def _fused_forward(x_nhwc, offset, mask, weight, bias, stride, padding, dilation,
                   bn_scale=None, bn_shift=None, act_relu=False):
    """out [B,Ho,Wo,Cout] = deformable conv of x with `offset` (2T, or raw 3T y) via the
    fused kernel; optional FrozenBN affine + ReLU folded into weight/bias and output."""
    B, H, W, Cin = x_nhwc.shape
    Cout, _, kH, kW = weight.shape
    Ho = out_size(H, padding, dilation, kH, stride)
    Wo = out_size(W, padding, dilation, kW, stride)
    dt = x_nhwc.dtype
    w = weight
    b = bias
    if bn_scale is not None:
        # relu(scale * (conv + bias) + shift) == relu(conv_{w*scale} + shift + scale*bias)
        w = weight * bn_scale.to(weight.dtype).view(-1, 1, 1, 1)
        b = bn_shift + (bias.to(bn_shift.dtype) * bn_scale if bias is not None else 0)
    b = b.to(dt).contiguous() if b is not None else None
    out = torch.empty(B, Ho, Wo, Cout, device=x_nhwc.device, dtype=dt)
    vec = 16 // x_nhwc.element_size()
    if Cin % vec == 0 and dt != torch.float64:
        # the BN-folded weight is a fresh tensor each call: pack it without caching
        w_packed = pack_weight(w, dt) if bn_scale is not None else packed_weight(w, dt)
        _ext().dcn_fused_fwd_nhwc(
            x_nhwc.contiguous(), offset.contiguous(),
            (mask if mask is not None else offset).contiguous(), w_packed, b, B, Cin, H, W,
            Ho, Wo, Cout, kH, kW, padding, padding, stride, stride, dilation, dilation, out)
    else:
        col = gather_cols_nhwc(x_nhwc, offset, mask, kH, kW, stride, padding, dilation)
        w_flat = w.permute(0, 2, 3, 1).to(dt).contiguous().view(Cout, kH * kW * Cin).t()
        torch.mm(col, w_flat, out=out.view(-1, Cout))
        if b is not None:
            out += b.view(1, 1, 1, -1)
    if bn_scale is not None and act_relu:
        out = torch.relu_(out)
    return out


def dcn_split_forward_nhwc(x_nhwc, w_off, b_off, weight, bias=None, stride=1, padding=1,
                           dilation=1):
    """Forward only: offset conv (library conv), then the fused deformable kernel."""
    y = F.conv2d(x_nhwc.permute(0, 3, 1, 2), w_off, b_off, stride, padding, dilation)
    y = y.permute(0, 2, 3, 1).contiguous()                 # [B,Ho,Wo,3T]
    return _fused_forward(x_nhwc, y, None, weight, bias, stride, padding, dilation)


class DCNSplitNHWCFunction(torch.autograd.Function):
    """NHWC DCNv2 with the offset conv inside.

    Inputs: x_nhwc [B,H,W,Cin], w_off [3T,Cin,kH,kW], b_off [3T], weight
    [Cout,Cin,kH,kW], bias [Cout] or None, stride, padding, dilation, and an optional
    FrozenBN epilogue (bn_scale, bn_shift per output channel; act_relu). Output
    [B,Ho,Wo,Cout]. Backward is not part of this build."""

    @staticmethod
    def forward(ctx, x_nhwc, w_off, b_off, weight, bias, stride, padding, dilation,
                bn_scale=None, bn_shift=None, act_relu=False):
        y = F.conv2d(x_nhwc.permute(0, 3, 1, 2), w_off, b_off, stride, padding, dilation)
        y = y.permute(0, 2, 3, 1).contiguous()
        return _fused_forward(x_nhwc, y, None, weight, bias, stride, padding, dilation,
                              bn_scale, bn_shift, act_relu)

    @staticmethod
    def backward(ctx, grad_out):
        raise RuntimeError("DCNSplitNHWCFunction.backward: the backward kernels are not part "
                           "of this build (forward operators only)")


def dcn_split_nhwc(x_nhwc, w_off, b_off, weight, bias=None, stride=1, padding=1, dilation=1,
                   bn_scale=None, bn_shift=None, act_relu=False):
    """NHWC DCNv2 forward with the offset conv inside; optional FrozenBN(+ReLU) epilogue."""
    return DCNSplitNHWCFunction.apply(x_nhwc, w_off, b_off, weight, bias, stride, padding,
                                      dilation, bn_scale, bn_shift, act_relu)


def _as_int(v):
    return v[0] if isinstance(v, (tuple, list)) else v


def dcn_apply_nchw(x_nchw, w_off, b_off, weight, bias=None, stride=1, padding=1, dilation=1,
                   bn_scale=None, bn_shift=None, act_relu=False):
    """NCHW-in / NCHW-out adapter over the NHWC path. A channels_last input is a free
    NHWC view and the output keeps the input's memory format."""
    s, p, d = _as_int(stride), _as_int(padding), _as_int(dilation)
    is_cl = x_nchw.is_contiguous(memory_format=torch.channels_last)
    x_nhwc = x_nchw.permute(0, 2, 3, 1)
    if not is_cl:
        x_nhwc = x_nhwc.contiguous()
    out_nhwc = dcn_split_nhwc(x_nhwc, w_off, b_off, weight, bias, s, p, d, bn_scale, bn_shift,
                              act_relu)
    out = out_nhwc.permute(0, 3, 1, 2)
    return out if is_cl else out.contiguous()
