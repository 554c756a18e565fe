"""Fused NHWC DCNv2 with the public names of naotic/bev-kernels
modulated_deform_conv/fused_tl.py, running on the gfx950 kernels of libbevk.so.

The reference builds these on TileLang JIT kernels; here every entry point runs on the
hand-written kernels: the deformable bilinear x mask taps are produced straight into LDS
tiles and multiplied on the matrix cores, so the [M, K] column matrix never reaches HBM;
the offset conv runs on the matrix cores too (fp32 accumulation), inside the same kernel
for the single-kernel forward. The backward (dcn_col2im_nhwc, dcn_split) runs the NHWC
column-to-image kernels.

Layout:
  data_im  [B, H, W, Cin]
  offset   [B, Ho, Wo, 2T]  (dy, dx per tap, T = kH*kW)
  mask     [B, Ho, Wo, T]
  weight   [Cout, Cin, kH, kW] (module layout; K order k = (ki*kW + kj)*Cin + ci)
  output   [B, Ho, Wo, Cout]
GEMM dims: M = B*Ho*Wo, N = Cout, K = kH*kW*Cin. groups == 1, deform_groups == 1.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import dcn_split_nhwc as _split
from ._packing import pack_weight


def out_size(H, pad, dil, k, stride):
    return (H + 2 * pad - (dil * (k - 1) + 1)) // stride + 1


def _triple(stride, padding, dilation):
    def two(v):
        return (v, v) if isinstance(v, int) else tuple(v)
    return two(stride), two(padding), two(dilation)


def _ext():
    import _modulated_deform_conv_ext as ext
    return ext


# ---------------------------------------------------------------------------------------
# Pure-PyTorch NHWC implementation (fused_tl.py:146-227 names); any device.
# ---------------------------------------------------------------------------------------

def _bilinear_nhwc(im_b, h, w):
    """im_b [H,W,Cin]; h, w [P] float coordinates -> [P, Cin]; neighbours outside the
    image count as zero and the whole sample is zero unless -1 < h < H, -1 < w < W."""
    H, W, Cin = im_b.shape
    hl = torch.floor(h)
    wl = torch.floor(w)
    lh, lw = h - hl, w - wl
    hh, hw = 1.0 - lh, 1.0 - lw
    hl, wl = hl.long(), wl.long()
    inside = ((h > -1) & (w > -1) & (h < H) & (w < W)).to(im_b.dtype)
    out = 0.0
    for dy, dx, wgt in ((0, 0, hh * hw), (0, 1, hh * lw), (1, 0, lh * hw), (1, 1, lh * lw)):
        y, x = hl + dy, wl + dx
        ok = ((y >= 0) & (y <= H - 1) & (x >= 0) & (x <= W - 1)).to(im_b.dtype)
        val = im_b[y.clamp(0, H - 1), x.clamp(0, W - 1)]
        out = out + (wgt * ok).unsqueeze(-1) * val
    return out * inside.unsqueeze(-1)


def dcn_columns_golden_nhwc(data_im, offset, mask, kH, kW, sh, sw, ph, pw, dh, dw):
    """Columns [B*Ho*Wo, T*Cin] (k = t*Cin + ci) in plain PyTorch."""
    B, H, W, Cin = data_im.shape
    Tt = kH * kW
    Ho = out_size(H, ph, dh, kH, sh)
    Wo = out_size(W, pw, dw, kW, sw)
    dev, dt = data_im.device, data_im.dtype
    oh = torch.arange(Ho, device=dev).view(Ho, 1).expand(Ho, Wo).reshape(-1)
    ow = torch.arange(Wo, device=dev).view(1, Wo).expand(Ho, Wo).reshape(-1)
    cols = data_im.new_zeros(B, Ho * Wo, Tt, Cin)
    for b in range(B):
        for t in range(Tt):
            ki, kj = divmod(t, kW)
            h = (oh * sh - ph + ki * dh).to(dt) + offset[b, :, :, 2 * t].reshape(-1)
            w = (ow * sw - pw + kj * dw).to(dt) + offset[b, :, :, 2 * t + 1].reshape(-1)
            cols[b, :, t, :] = _bilinear_nhwc(data_im[b], h, w) * mask[b, :, :, t].reshape(-1, 1)
    return cols.reshape(B * Ho * Wo, Tt * Cin)


def dcn_forward_golden_nhwc(data_im, offset, mask, weight, bias=None, stride=1, padding=0,
                            dilation=1):
    """NHWC forward [B,Ho,Wo,Cout] in plain PyTorch."""
    (sh, sw), (ph, pw), (dh, dw) = _triple(stride, padding, dilation)
    B, H, W, Cin = data_im.shape
    Cout, _, kH, kW = weight.shape
    Ho = out_size(H, ph, dh, kH, sh)
    Wo = out_size(W, pw, dw, kW, sw)
    cols = dcn_columns_golden_nhwc(data_im, offset, mask, kH, kW, sh, sw, ph, pw, dh, dw)
    out = (cols @ weight.permute(2, 3, 1, 0).reshape(kH * kW * Cin, Cout)).view(B, Ho, Wo, Cout)
    if bias is not None:
        out = out + bias.view(1, 1, 1, -1)
    return out


# ---------------------------------------------------------------------------------------
# Kernel-backed entry points
# ---------------------------------------------------------------------------------------

def weight_to_nhwc_flat(weight, block_K=32):
    """torch weight [Cout,Cin,kH,kW] -> [Kpad, Cout], k = (ki*kW+kj)*Cin+ci (zero rows
    pad K to a multiple of block_K)."""
    Cout, Cin, kH, kW = weight.shape
    K = kH * kW * Cin
    w_flat = weight.permute(2, 3, 1, 0).reshape(K, Cout).contiguous()
    Kpad = ((K + block_K - 1) // block_K) * block_K
    if Kpad != K:
        w_pad = w_flat.new_zeros(Kpad, Cout)
        w_pad[:K] = w_flat
        w_flat = w_pad
    return w_flat


def _check_single_group(data_im, weight):
    if weight.size(1) != data_im.size(-1):
        raise RuntimeError("groups>1 not supported in fused_tl")


def fused_dcn_forward_nhwc(data_im, offset, mask, weight, bias=None, stride=1, padding=0,
                           dilation=1, block_M=32, block_N=256, block_K=32, num_stages=2,
                           threads=256, return_flat=False):
    """Forward modulated deformable conv2d (groups=1, dg=1), NHWC, on the fused kernel.

    data_im [B,H,W,Cin], offset [B,Ho,Wo,2T], mask [B,Ho,Wo,T], weight [Cout,Cin,kH,kW],
    bias [Cout] or None -> out [B,Ho,Wo,Cout] (or [B*Ho*Wo, Cout] with return_flat).
    The block_* / num_stages / threads arguments of the TileLang version are accepted
    and ignored: tiles are chosen by the kernel."""
    (sh, sw), (ph, pw), (dh, dw) = _triple(stride, padding, dilation)
    _check_single_group(data_im, weight)
    B, H, W, Cin = data_im.shape
    Cout, _, kH, kW = weight.shape
    Ho = out_size(H, ph, dh, kH, sh)
    Wo = out_size(W, pw, dw, kW, sw)
    dt = data_im.dtype
    out = torch.empty(B, Ho, Wo, Cout, device=data_im.device, dtype=dt)
    b = bias.to(dt).contiguous() if bias is not None else None
    vec = 16 // data_im.element_size()
    if Cin % vec == 0 and dt != torch.float64:
        _ext().dcn_fused_fwd_nhwc(data_im.contiguous(), offset.contiguous(), mask.contiguous(),
                                  pack_weight(weight, dt), b, B, Cin, H, W, Ho, Wo, Cout, kH, kW, ph, pw, sh, sw,
                                  dh, dw, out)
    else:
        cols = dcn_gather_cols_nhwc(data_im, offset, mask, kH, kW, (sh, sw), (ph, pw), (dh, dw))
        w_kc = weight.permute(0, 2, 3, 1).to(dt).contiguous()
        torch.mm(cols, w_kc.view(Cout, -1).t(), out=out.view(-1, Cout))
        if b is not None:
            out += b.view(1, 1, 1, -1)
    return out.view(B * Ho * Wo, Cout) if return_flat else out


def dcn_gather_cols_nhwc(data_im, offset, mask, kH, kW, stride=1, padding=0, dilation=1,
                         block_M=64, block_K=64, threads=256):
    """Deformable gather -> columns [M, K] (NHWC, k = t*Cin+ci)."""
    (sh, sw), (ph, pw), (dh, dw) = _triple(stride, padding, dilation)
    B, H, W, Cin = data_im.shape
    Ho = out_size(H, ph, dh, kH, sh)
    Wo = out_size(W, pw, dw, kW, sw)
    M = B * Ho * Wo
    cols = torch.empty(M, kH * kW * Cin, device=data_im.device, dtype=data_im.dtype)
    _ext().modulated_deformable_im2col_nhwc_cuda(
        data_im.contiguous(), offset.contiguous(), mask.contiguous(), B, Cin, H, W, Ho, Wo, kH,
        kW, ph, pw, sh, sw, dh, dw, 1, cols)
    return cols


def offset_conv_forward_nhwc(data_im, w_off, b_off, kH, kW, stride=1, padding=0, dilation=1,
                             block_M=64, block_N=32, block_K=32, num_stages=2, threads=256):
    """Offset conv -> (offset [B,Ho,Wo,2T], mask [B,Ho,Wo,T]) in the input dtype, as
    mmcv's Pack splits it (fused_tl.py:419-470): y = conv(x, w_off) + b_off accumulated
    and kept in fp32 (the matrix-core kernel dcn_offset_conv_nhwc), offset = y[..., :2T],
    mask = sigmoid(y[..., 2T:3T]), both rounded once to the input dtype. The block_* /
    num_stages / threads arguments of the TileLang version are accepted and ignored."""
    Tt = kH * kW
    if w_off.size(0) != 3 * Tt or w_off.size(1) != data_im.size(-1):
        raise RuntimeError("offset conv weight must be [3*kH*kW, Cin, kH, kW]")
    dt = data_im.dtype
    if _split.offset_conv_supported(data_im, w_off):
        y = _split.offset_conv_y(data_im, w_off, b_off, stride, padding, dilation)
    else:
        (sh, sw), (ph, pw), (dh, dw) = _triple(stride, padding, dilation)
        y = F.conv2d(data_im.permute(0, 3, 1, 2).float(), w_off.float(),
                     b_off.float() if b_off is not None else None, (sh, sw), (ph, pw),
                     (dh, dw)).permute(0, 2, 3, 1)
    offset = y[..., :2 * Tt].to(dt).contiguous()
    mask = torch.sigmoid(y[..., 2 * Tt:]).to(dt).contiguous()
    return offset, mask


def dcn_forward_split_nhwc(data_im, w_off, b_off, weight, bias=None, stride=1, padding=0,
                           dilation=1):
    """Full DCNv2 forward (NHWC, groups=1, dg=1; fused_tl.py:373-403): offset conv and the
    deformable conv in one kernel (the offsets stay fp32 between them)."""
    _check_single_group(data_im, weight)
    if _split.mega_supported(data_im, w_off, weight):
        return _split.mega_forward(data_im, w_off, b_off, weight, bias, stride, padding,
                                   dilation)[0]
    offset, mask = offset_conv_forward_nhwc(data_im, w_off, b_off, weight.size(2),
                                            weight.size(3), stride, padding, dilation)
    return fused_dcn_forward_nhwc(data_im, offset, mask, weight, bias, stride, padding,
                                  dilation)


def fused_dcn_full_forward_nhwc(data_im, w_off, b_off, weight, bias=None, stride=1, padding=0,
                                dilation=1):
    """Full DCNv2 forward (NHWC) as the reference composes it (fused_tl.py:473-484): the
    offset conv (offset and mask rounded to the input dtype), then the fused deformable
    kernel."""
    _, _, kH, kW = weight.shape
    offset, mask = offset_conv_forward_nhwc(data_im, w_off, b_off, kH, kW, stride, padding,
                                            dilation)
    return fused_dcn_forward_nhwc(data_im, offset, mask, weight, bias, stride, padding,
                                  dilation)


def fused_dcn_mega_forward_nhwc(data_im, w_off, b_off, weight, bias=None, stride=1, padding=0,
                                dilation=1, block_M=32, block_N=None, block_K=64, num_stages=2,
                                threads=256):
    """Single-kernel full DCNv2 forward (NHWC, groups=1, dg=1; fused_tl.py:565-766): offset
    conv (fp32 accumulation, kept in fp32), sigmoid, deformable gather and main GEMM in one
    launch on the persistent fp16/bf16 kernel (two launches on other shapes)."""
    _check_single_group(data_im, weight)
    if not _split.mega_supported(data_im, w_off, weight):
        return dcn_forward_split_nhwc(data_im, w_off, b_off, weight, bias, stride, padding,
                                      dilation)
    return _split.mega_forward(data_im, w_off, b_off, weight, bias, stride, padding,
                               dilation)[0]


def dcn_col2im_nhwc(dCol, X, offset, mask, kH, kW, stride=1, padding=0, dilation=1, block=256):
    """Backward column-to-image (fused_tl.py:792-862): dCol [M, T*Cin], X [B,H,W,Cin],
    offset [B,Ho,Wo,2T], mask [B,Ho,Wo,T] -> (grad_X [B,H,W,Cin], grad_offset
    [B,Ho,Wo,2T], grad_mask [B,Ho,Wo,T]), all float32, computed in fp32 on fp32 copies of
    the inputs as the reference does. `block` is accepted and ignored."""
    (sh, sw), (ph, pw), (dh, dw) = _triple(stride, padding, dilation)
    B, H, W, Cin = X.shape
    Ho = out_size(H, ph, dh, kH, sh)
    Wo = out_size(W, pw, dw, kW, sw)
    Tt = kH * kW
    dev = X.device
    gX = torch.zeros(B, H, W, Cin, device=dev, dtype=torch.float32)
    gOff = torch.empty(B, Ho, Wo, 2 * Tt, device=dev, dtype=torch.float32)
    gMask = torch.empty(B, Ho, Wo, Tt, device=dev, dtype=torch.float32)
    _ext().modulated_deformable_col2im_nhwc_cuda(
        dCol.float().contiguous(), X.float().contiguous(), offset.float().contiguous(),
        mask.float().contiguous(), B, Cin, H, W, Ho, Wo, kH, kW, ph, pw, sh, sw, dh, dw, 1, gX,
        gOff, gMask)
    return gX, gOff, gMask


class _DCNSplitFunction(torch.autograd.Function):
    """Differentiable full DCNv2 (NHWC; fused_tl.py:866-943): forward = the one-kernel
    forward, backward = the NHWC split composition (re-gathered columns, dCol = dO @ W,
    column-to-image kernel, library offset-conv backward)."""

    @staticmethod
    def forward(ctx, x_nhwc, w_off, b_off, weight, bias, stride, padding, dilation):
        (sh, sw), (ph, pw), (dh, dw) = _triple(stride, padding, dilation)
        if sh != sw or ph != pw or dh != dw:
            raise RuntimeError("dcn_split needs uniform stride/padding/dilation")
        _check_single_group(x_nhwc, weight)
        out, y = _split._split_forward(x_nhwc, w_off, b_off, weight, bias, sh, ph, dh)
        ctx.save_for_backward(x_nhwc, y, w_off, weight)
        ctx.stride, ctx.padding, ctx.dilation = sh, ph, dh
        ctx.with_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, y, w_off, weight = ctx.saved_tensors
        grads = _split.split_backward(grad_out, x, y, w_off, weight, ctx.stride, ctx.padding,
                                      ctx.dilation, ctx.with_bias)
        return grads + (None, None, None)


def dcn_split(x_nhwc, w_off, b_off, weight, bias=None, stride=1, padding=0, dilation=1):
    """Autograd-enabled full DCNv2 forward (NHWC)."""
    return _DCNSplitFunction.apply(x_nhwc, w_off, b_off, weight, bias, stride, padding, dilation)


def dcn_apply_nchw(x_nchw, w_off, b_off, weight, bias=None, stride=1, padding=0, dilation=1):
    """NCHW-in / NCHW-out adapter over the NHWC forward; channels_last input is a free
    NHWC view and the output keeps the input's memory format."""
    is_cl = x_nchw.is_contiguous(memory_format=torch.channels_last)
    x_nhwc = x_nchw.permute(0, 2, 3, 1)
    if not is_cl:
        x_nhwc = x_nhwc.contiguous()
    out_nhwc = dcn_split(x_nhwc, w_off, b_off, weight, bias, stride, padding, dilation)
    out = out_nhwc.permute(0, 3, 1, 2)
    return out if is_cl else out.contiguous()
