"""NHWC DCNv2: offset conv + deformable gather/GEMM, with the public names of
naotic/bev-kernels modulated_deform_conv/dcn_split_nhwc.py.

Layout: x [B,H,W,Cin], w_off [3T,Cin,kH,kW], b_off [3T], weight [Cout,Cin,kH,kW];
output [B,Ho,Wo,Cout].

The forward is one gfx950 kernel (_modulated_deform_conv_ext.dcn_mega_fwd_nhwc): the
offset conv runs on the matrix cores with fp32 accumulation, its output y [B,Ho,Wo,3T]
(offsets, then the pre-sigmoid mask; kept in fp32) feeds the deformable taps, which are
built in LDS and multiplied on the matrix cores, and the FrozenBN + ReLU epilogue is
folded into the weight, the bias and the kernel's store. Neither the [M, T*Cin] column
matrix nor a library convolution is involved; y is written once (float32) for the
backward. ``gather_cols_nhwc`` still materialises the columns for callers that want them.
Shapes the kernels do not take (float64, channel counts that are not a multiple of 16
bytes) use the library offset conv and the column path.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from ._packing import pack_weight


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


def _pair(v):
    return (v, v) if isinstance(v, int) else (int(v[0]), int(v[1]))


def _fold_bn(weight, bias, bn_scale, bn_shift):
    """relu(scale * (conv_w(x) + bias) + shift) == relu(conv_{w*scale}(x) + shift +
    scale*bias) for per-output-channel FrozenBN (dcn_split_nhwc.py:178-204)."""
    if bn_scale is None:
        return weight, bias
    w = weight * bn_scale.to(weight.dtype).view(-1, 1, 1, 1)
    b = bn_shift + (bias.to(bn_shift.dtype) * bn_scale if bias is not None else 0)
    return w, b


def _fused_forward(x_nhwc, offset, mask, weight, bias, stride, padding, dilation,
                   bn_scale=None, bn_shift=None, act_relu=False):
    """out [B,Ho,Wo,Cout] = deformable conv of x with `offset` (2T, or raw 3T y) via the
    fused kernel; optional FrozenBN affine + ReLU folded into weight/bias and output."""
    B, H, W, Cin = x_nhwc.shape
    Cout, _, kH, kW = weight.shape
    Ho = out_size(H, padding, dilation, kH, stride)
    Wo = out_size(W, padding, dilation, kW, stride)
    dt = x_nhwc.dtype
    w, b = _fold_bn(weight, bias, bn_scale, bn_shift)
    b = b.to(dt).contiguous() if b is not None else None
    out = torch.empty(B, Ho, Wo, Cout, device=x_nhwc.device, dtype=dt)
    vec = 16 // x_nhwc.element_size()
    if Cin % vec == 0 and dt != torch.float64:
        _ext().dcn_fused_fwd_nhwc(
            x_nhwc.contiguous(), offset.contiguous(),
            (mask if mask is not None else offset).contiguous(), pack_weight(w, dt), b, B, Cin,
            H, W, Ho, Wo, Cout, kH, kW, padding, padding, stride, stride, dilation, dilation,
            out)
    else:
        col = gather_cols_nhwc(x_nhwc, offset, mask, kH, kW, stride, padding, dilation)
        w_flat = w.permute(0, 2, 3, 1).to(dt).contiguous().view(Cout, kH * kW * Cin).t()
        torch.mm(col, w_flat, out=out.view(-1, Cout))
        if b is not None:
            out += b.view(1, 1, 1, -1)
    if bn_scale is not None and act_relu:
        out = torch.relu_(out)
    return out


def offset_conv_supported(x_nhwc, w_off):
    """True when the matrix-core offset conv (dcn_offset_conv_nhwc) takes x [B,H,W,Cin] and
    w_off [3T, Cin, kH, kW]: fp32 / fp16 / bf16, Cin a multiple of 16 bytes' worth of
    elements, at most 9 taps for the 16-bit types."""
    if x_nhwc.dtype not in (torch.float32, torch.float16, torch.bfloat16) or w_off.dim() != 4:
        return False
    n3, cin_w, kH, kW = w_off.shape
    cin = x_nhwc.shape[-1]
    vec = 16 // x_nhwc.element_size()
    return (n3 == 3 * kH * kW and cin_w == cin and cin % vec == 0
            and (x_nhwc.dtype == torch.float32 or kH * kW <= 9))


def mega_supported(x_nhwc, w_off, weight):
    """True when the one-kernel forward (dcn_mega_fwd_nhwc) takes these tensors."""
    return (offset_conv_supported(x_nhwc, w_off)
            and tuple(weight.shape[1:]) == tuple(w_off.shape[1:]))


def offset_conv_y(x_nhwc, w_off, b_off, stride=1, padding=1, dilation=1):
    """y [B,Ho,Wo,3T] float32 = conv(x, w_off) + b_off, fp32 accumulation on the matrix
    cores (dcn_offset_conv_nhwc); offset_conv_supported(x_nhwc, w_off) must hold."""
    (sh, sw), (ph, pw), (dh, dw) = _pair(stride), _pair(padding), _pair(dilation)
    B, H, W, Cin = x_nhwc.shape
    kH, kW = w_off.shape[2], w_off.shape[3]
    Ho, Wo = out_size(H, ph, dh, kH, sh), out_size(W, pw, dw, kW, sw)
    dt = x_nhwc.dtype
    y = torch.empty(B, Ho, Wo, 3 * kH * kW, device=x_nhwc.device, dtype=torch.float32)
    _ext().dcn_offset_conv_nhwc(
        x_nhwc.contiguous(), pack_weight(w_off, dt),
        b_off.float().contiguous() if b_off is not None else None, B, Cin, H, W, Ho, Wo, kH, kW,
        ph, pw, sh, sw, dh, dw, y)
    return y


def mega_forward(x_nhwc, w_off, b_off, weight, bias=None, stride=1, padding=1, dilation=1,
                 act_relu=False):
    """One-kernel forward: (out [B,Ho,Wo,Cout] in the input dtype, y [B,Ho,Wo,3T] float32
    = the offset conv with its bias, which the backward needs). mega_supported must hold."""
    (sh, sw), (ph, pw), (dh, dw) = _pair(stride), _pair(padding), _pair(dilation)
    B, H, W, Cin = x_nhwc.shape
    Cout, _, kH, kW = weight.shape
    Ho, Wo = out_size(H, ph, dh, kH, sh), out_size(W, pw, dw, kW, sw)
    dt = x_nhwc.dtype
    y = torch.empty(B, Ho, Wo, 3 * kH * kW, device=x_nhwc.device, dtype=torch.float32)
    out = torch.empty(B, Ho, Wo, Cout, device=x_nhwc.device, dtype=dt)
    _ext().dcn_mega_fwd_nhwc(
        x_nhwc.contiguous(), pack_weight(w_off, dt),
        b_off.float().contiguous() if b_off is not None else None, pack_weight(weight, dt),
        bias.to(dt).contiguous() if bias is not None else None, B, Cin, H, W, Ho, Wo, Cout,
        kH, kW, ph, pw, sh, sw, dh, dw, act_relu, y, out)
    return out, y


def _split_forward(x_nhwc, w_off, b_off, weight, bias, stride, padding, dilation,
                   bn_scale=None, bn_shift=None, act_relu=False):
    """(out, y): the one-kernel forward where it applies, else the library offset conv (y
    in the input dtype) and the fused / column path."""
    if mega_supported(x_nhwc, w_off, weight):
        w, b = _fold_bn(weight, bias, bn_scale, bn_shift)
        return mega_forward(x_nhwc, w_off, b_off, w, b, stride, padding, dilation,
                            act_relu=bn_scale is not None and act_relu)
    y = F.conv2d(x_nhwc.permute(0, 3, 1, 2), w_off, b_off, stride, padding, dilation)
    y = y.permute(0, 2, 3, 1).contiguous()                 # [B,Ho,Wo,3T]
    out = _fused_forward(x_nhwc, y, None, weight, bias, stride, padding, dilation, bn_scale,
                         bn_shift, act_relu)
    return out, y


def split_backward(grad_out, x, y, w_off, weight, stride, padding, dilation, with_bias,
                   bn_scale=None, relu_mask=None):
    """Backward of the NHWC split forward (dcn_split_nhwc.py:230-291): the columns are
    re-gathered from x and y (the reference's default DCN_RECOMPUTE_COLS=1), dCol = dO @ W,
    grad_weight = cols^T @ dO in fp32, the column-to-image kernel gives grad_x (samples),
    grad_offset and the pre-sigmoid grad_mask, and the offset conv's backward is the library
    convolution backward. y is the offset-conv output with bias (float32 or the input
    dtype); the kernels read it in the input dtype. Returns (grad_x, grad_w_off,
    grad_b_off, grad_weight, grad_bias)."""
    st, pd, dl = stride, padding, dilation
    Cout, _, kH, kW = weight.shape
    B, H, W, Cin = x.shape
    Ho = out_size(H, pd, dl, kH, st)
    Wo = out_size(W, pd, dl, kW, st)
    M, K = B * Ho * Wo, kH * kW * Cin
    dt = x.dtype
    y = y.to(dt).contiguous()

    go = grad_out.reshape(M, Cout)
    if relu_mask is not None:
        go = go * relu_mask.reshape(M, Cout)
    if bn_scale is not None:
        go = go * bn_scale.to(go.dtype).view(1, -1)
    dO = go.to(dt).contiguous()
    w_flat = weight.permute(2, 3, 1, 0).reshape(K, Cout).contiguous().to(dt)

    cols = gather_cols_nhwc(x, y, None, kH, kW, st, pd, dl)
    dCol = torch.mm(dO, w_flat.t())
    grad_weight = torch.mm(cols.t().float(), dO.float()) \
        .view(kH, kW, Cin, Cout).permute(3, 2, 0, 1).contiguous().to(weight.dtype)
    grad_bias = dO.float().sum(0).to(dt) if with_bias else None

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
            grad_bias)


def dcn_split_forward_nhwc(x_nhwc, w_off, b_off, weight, bias=None, stride=1, padding=1,
                           dilation=1):
    """Forward only (dcn_split_nhwc.py:117-147): offset conv, then the deformable conv, in
    one kernel where it applies."""
    return _split_forward(x_nhwc, w_off, b_off, weight, bias, stride, padding, dilation)[0]


class DCNSplitNHWCFunction(torch.autograd.Function):
    """NHWC DCNv2 with the offset conv inside (dcn_split_nhwc.py:150-291).

    Inputs: x_nhwc [B,H,W,Cin], w_off [3T,Cin,kH,kW], b_off [3T], weight
    [Cout,Cin,kH,kW], bias [Cout] or None, stride, padding, dilation, and an optional
    FrozenBN epilogue (bn_scale, bn_shift per output channel; act_relu). Output
    [B,Ho,Wo,Cout].

    Forward: one kernel (offset conv, sigmoid, deformable gather, GEMM, epilogue) where it
    applies; y is saved for the backward (split_backward)."""

    @staticmethod
    def forward(ctx, x_nhwc, w_off, b_off, weight, bias, stride, padding, dilation,
                bn_scale=None, bn_shift=None, act_relu=False):
        out, y = _split_forward(x_nhwc, w_off, b_off, weight, bias, stride, padding, dilation,
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
        saved = list(ctx.saved_tensors)
        x, y, w_off, weight = saved[:4]
        bn_scale = saved[4] if ctx.has_bn else None
        relu_mask = saved[5] if ctx.act_relu else None
        grads = split_backward(grad_out, x, y, w_off, weight, ctx.stride, ctx.padding,
                               ctx.dilation, ctx.with_bias, bn_scale, relu_mask)
        return grads + (None, None, None, None, None, None)


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
