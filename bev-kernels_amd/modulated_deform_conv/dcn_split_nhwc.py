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
    """Backward column-to-image (dcn_split_nhwc.py:48-114). Returns (grad_x_samp, grad_offset,
    grad_mask), all float32. With mask=None, `offset` is the raw offset-conv output
    y [B,Ho,Wo,3T] and grad_mask is the gradient of the pre-sigmoid mask (sigmoid backward
    folded in), as the reference's per-element kernels return it. The reference's
    DCN_COL2IM_MODE kernel choice has one kernel here."""
    B, H, W, Cin = x_nhwc.shape
    Tt = kH * kW
    Ho = out_size(H, padding, dilation, kH, stride)
    Wo = out_size(W, padding, dilation, kW, stride)
    dev = x_nhwc.device
    gX = torch.zeros(B, H, W, Cin, device=dev, dtype=torch.float32)
    gOff = torch.empty(B, Ho, Wo, 2 * Tt, device=dev, dtype=torch.float32)
    gMask = torch.empty(B, Ho, Wo, Tt, device=dev, dtype=torch.float32)
    off_c = offset.contiguous()
    _ext().modulated_deformable_col2im_nhwc_cuda(
        dcol.contiguous(), x_nhwc.contiguous(), off_c,
        (mask if mask is not None else off_c).contiguous(), B, Cin, H, W, Ho, Wo, kH, kW,
        padding, padding, stride, stride, dilation, dilation, 1, gX, gOff, gMask)
    return gX, gOff, gMask


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
    """NHWC DCNv2 with the offset conv inside (dcn_split_nhwc.py:150-291).

    Inputs: x_nhwc [B,H,W,Cin], w_off [3T,Cin,kH,kW], b_off [3T], weight
    [Cout,Cin,kH,kW], bias [Cout] or None, stride, padding, dilation, and an optional
    FrozenBN epilogue (bn_scale, bn_shift per output channel; act_relu). Output
    [B,Ho,Wo,Cout].

    Forward: library offset conv, then the fused deformable kernel on its raw output y.
    Backward (the reference's composition): the columns are re-gathered from x and y (the
    reference's default DCN_RECOMPUTE_COLS=1), dCol = dO @ W, grad_weight = cols^T @ dO in
    fp32, the column-to-image kernel gives grad_x (samples), grad_offset and the pre-sigmoid
    grad_mask, and the offset conv's backward is the library convolution backward."""

    @staticmethod
    def forward(ctx, x_nhwc, w_off, b_off, weight, bias, stride, padding, dilation,
                bn_scale=None, bn_shift=None, act_relu=False):
        y = F.conv2d(x_nhwc.permute(0, 3, 1, 2), w_off, b_off, stride, padding, dilation)
        y = y.permute(0, 2, 3, 1).contiguous()
        out = _fused_forward(x_nhwc, y, None, weight, bias, stride, padding, dilation,
                             bn_scale, bn_shift, act_relu)
        ctx.has_bn = bn_scale is not None
        ctx.act_relu = bool(act_relu) and ctx.has_bn
        saved = [x_nhwc, y, w_off, weight]
        if ctx.has_bn:
            saved.append(bn_scale)
            if ctx.act_relu:
                saved.append(out > 0)
        ctx.save_for_backward(*saved)
        ctx.stride, ctx.padding, ctx.dilation = stride, padding, dilation
        ctx.with_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, grad_out):
        st, pd, dl = ctx.stride, ctx.padding, ctx.dilation
        saved = list(ctx.saved_tensors)
        x, y, w_off, weight = saved[:4]
        bn_scale = saved[4] if ctx.has_bn else None
        relu_mask = saved[5] if ctx.act_relu else None
        Cout, _, kH, kW = weight.shape
        B, H, W, Cin = x.shape
        Ho = out_size(H, pd, dl, kH, st)
        Wo = out_size(W, pd, dl, kW, st)
        M, K = B * Ho * Wo, kH * kW * Cin
        dt = x.dtype

        go = grad_out.reshape(M, Cout)
        if ctx.has_bn:
            if ctx.act_relu:
                go = go * relu_mask.reshape(M, Cout)
            go = go * bn_scale.to(go.dtype).view(1, -1)
        dO = go.to(dt).contiguous()
        w_flat = weight.permute(2, 3, 1, 0).reshape(K, Cout).contiguous().to(dt)

        cols = gather_cols_nhwc(x, y, None, kH, kW, st, pd, dl)
        dCol = torch.mm(dO, w_flat.t())
        grad_weight = torch.mm(cols.t().float(), dO.float()) \
            .view(kH, kW, Cin, Cout).permute(3, 2, 0, 1).contiguous().to(weight.dtype)
        grad_bias = dO.float().sum(0).to(dt) if ctx.with_bias else None

        gX_samp, gOff, gmask_raw = col2im_nhwc(dCol, x, y, None, kH, kW, st, pd, dl)

        dY = torch.cat([gOff, gmask_raw], dim=-1).permute(0, 3, 1, 2).contiguous()
        x_nchw = x.permute(0, 3, 1, 2).contiguous().float()
        w_off_f = w_off.float()
        s2, p2, d2 = (st, st), (pd, pd), (dl, dl)
        grad_x_off = torch.nn.grad.conv2d_input(x_nchw.shape, w_off_f, dY, s2, p2, d2)
        grad_w_off = torch.nn.grad.conv2d_weight(x_nchw, w_off_f.shape, dY, s2, p2, d2)
        grad_b_off = dY.sum(dim=(0, 2, 3))
        grad_x = (gX_samp + grad_x_off.permute(0, 2, 3, 1)).to(dt)
        return (grad_x, grad_w_off.to(w_off.dtype), grad_b_off.to(w_off.dtype), grad_weight,
                grad_bias, None, None, None, None, None, None)


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
