"""Modulated deformable conv2d (DCNv2): extension wrappers, modules and a pure-PyTorch
implementation, with the public names of naotic/bev-kernels
modulated_deform_conv/modulated_deform_conv.py.

Forward runs on the gfx950 kernels of libbevk.so (through ``_modulated_deform_conv_ext``).
Backward: ModulatedDeformConv2dFunction.backward follows the reference's composition
(modulated_deform_conv.py:405-500) on the NCHW column-to-image kernel.
"""
from __future__ import annotations

import math
import os

import torch
import torch.nn as nn
from torch.autograd import Function
from torch.autograd.function import once_differentiable
from torch.nn.modules.utils import _pair, _single
from ._packing import pack_weight

_ext = None


def _load_ext():
    global _ext
    if _ext is None:
        import _modulated_deform_conv_ext as ext
        _ext = ext
    return _ext


def _out_size(size, pad, dil, k, stride):
    return (size + 2 * pad - (dil * (k - 1) + 1)) // stride + 1


# ---------------------------------------------------------------------------------------
# Extension wrappers (modulated_deform_conv.py:30-177)
# ---------------------------------------------------------------------------------------

def ext_modulated_deformable_im2col(data_im, data_offset, data_mask, kernel_h, kernel_w,
                                    pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                                    deformable_group):
    """Columns [C*kh*kw, B, Ho, Wo] of the NCHW input (per-channel kernel)."""
    ext = _load_ext()
    batch_size, channels, height, width = data_im.shape
    height_col = _out_size(height, pad_h, dilation_h, kernel_h, stride_h)
    width_col = _out_size(width, pad_w, dilation_w, kernel_w, stride_w)
    # Every element is written by the kernel: no zero fill needed.
    data_col = data_im.new_empty(channels * kernel_h * kernel_w, batch_size, height_col,
                                 width_col)
    ext.modulated_deformable_im2col_cuda(
        data_im, data_offset, data_mask, batch_size, channels, height, width, height_col,
        width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
        deformable_group, data_col)
    return data_col


def ext_modulated_deformable_im2col_opt(data_im, data_offset, data_mask, kernel_h, kernel_w,
                                        pad_h, pad_w, stride_h, stride_w, dilation_h,
                                        dilation_w, deformable_group):
    """Columns [C*kh*kw, B, Ho, Wo] of the NCHW input (geometry-reuse kernel)."""
    ext = _load_ext()
    batch_size, channels, height, width = data_im.shape
    height_col = _out_size(height, pad_h, dilation_h, kernel_h, stride_h)
    width_col = _out_size(width, pad_w, dilation_w, kernel_w, stride_w)
    data_col = data_im.new_empty(channels * kernel_h * kernel_w, batch_size, height_col,
                                 width_col)
    ext.modulated_deformable_im2col_opt_cuda(
        data_im, data_offset, data_mask, batch_size, channels, height, width, height_col,
        width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
        deformable_group, data_col)
    return data_col


def _col2im_common(entry, data_col, data_offset, data_mask, batch_size, channels, height,
                   width, kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h,
                   dilation_w, deformable_group):
    ext = _load_ext()
    height_col = _out_size(height, pad_h, dilation_h, kernel_h, stride_h)
    width_col = _out_size(width, pad_w, dilation_w, kernel_w, stride_w)
    grad_im = data_col.new_zeros(batch_size, channels, height, width)
    getattr(ext, entry)(data_col, data_offset, data_mask, batch_size, channels, height, width,
                        height_col, width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h,
                        stride_w, dilation_h, dilation_w, deformable_group, grad_im)
    return grad_im


def ext_modulated_deformable_col2im_opt(data_col, data_offset, data_mask, batch_size, channels,
                                        height, width, kernel_h, kernel_w, pad_h, pad_w,
                                        stride_h, stride_w, dilation_h, dilation_w,
                                        deformable_group):
    return _col2im_common("modulated_deformable_col2im_opt_cuda", data_col, data_offset,
                          data_mask, batch_size, channels, height, width, kernel_h, kernel_w,
                          pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                          deformable_group)


def ext_modulated_deformable_col2im_smem(data_col, data_offset, data_mask, batch_size,
                                         channels, height, width, kernel_h, kernel_w, pad_h,
                                         pad_w, stride_h, stride_w, dilation_h, dilation_w,
                                         deformable_group):
    return _col2im_common("modulated_deformable_col2im_smem_cuda", data_col, data_offset,
                          data_mask, batch_size, channels, height, width, kernel_h, kernel_w,
                          pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                          deformable_group)


def ext_modulated_deformable_col2im(data_col, data_offset, data_mask, batch_size, channels,
                                    height, width, kernel_h, kernel_w, pad_h, pad_w, stride_h,
                                    stride_w, dilation_h, dilation_w, deformable_group):
    return _col2im_common("modulated_deformable_col2im_cuda", data_col, data_offset, data_mask,
                          batch_size, channels, height, width, kernel_h, kernel_w, pad_h, pad_w,
                          stride_h, stride_w, dilation_h, dilation_w, deformable_group)


def _col2im_coord_common(entry, data_col, data_im, data_offset, data_mask, kernel_h, kernel_w,
                         pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                         deformable_group):
    ext = _load_ext()
    batch_size, channels, height, width = data_im.shape
    height_col = _out_size(height, pad_h, dilation_h, kernel_h, stride_h)
    width_col = _out_size(width, pad_w, dilation_w, kernel_w, stride_w)
    grad_offset = data_offset.new_zeros(data_offset.shape)
    grad_mask = data_mask.new_zeros(data_mask.shape)
    getattr(ext, entry)(data_col, data_im, data_offset, data_mask, batch_size, channels, height,
                        width, height_col, width_col, kernel_h, kernel_w, pad_h, pad_w,
                        stride_h, stride_w, dilation_h, dilation_w, deformable_group,
                        grad_offset, grad_mask)
    return grad_offset, grad_mask


def ext_modulated_deformable_col2im_coord(data_col, data_im, data_offset, data_mask, kernel_h,
                                          kernel_w, pad_h, pad_w, stride_h, stride_w,
                                          dilation_h, dilation_w, deformable_group):
    return _col2im_coord_common("modulated_deformable_col2im_coord_cuda", data_col, data_im,
                                data_offset, data_mask, kernel_h, kernel_w, pad_h, pad_w,
                                stride_h, stride_w, dilation_h, dilation_w, deformable_group)


def ext_modulated_deformable_col2im_coord_opt(data_col, data_im, data_offset, data_mask,
                                              kernel_h, kernel_w, pad_h, pad_w, stride_h,
                                              stride_w, dilation_h, dilation_w,
                                              deformable_group):
    return _col2im_coord_common("modulated_deformable_col2im_coord_opt_cuda", data_col, data_im,
                                data_offset, data_mask, kernel_h, kernel_w, pad_h, pad_w,
                                stride_h, stride_w, dilation_h, dilation_w, deformable_group)


# ---------------------------------------------------------------------------------------
# Pure-PyTorch implementation (differentiable, any device): the columns that the kernels
# produce, built from whole-channel gathers. Not used by the operators above.
# ---------------------------------------------------------------------------------------

def _bilinear_sample(data_im_ptr, height, width, h, w):
    """Bilinear sample of a [H, W] plane at float coordinates h, w ([N] each); each of
    the four neighbours counts as zero outside the plane."""
    h_low = h.floor()
    w_low = w.floor()
    lh = h - h_low
    lw = w - w_low
    hh = 1.0 - lh
    hw = 1.0 - lw
    h_low = h_low.long()
    w_low = w_low.long()

    def corner(iy, ix):
        inside = (iy >= 0) & (iy <= height - 1) & (ix >= 0) & (ix <= width - 1)
        val = data_im_ptr[iy.clamp(0, height - 1), ix.clamp(0, width - 1)]
        return val * inside.to(val.dtype)

    return (hh * hw * corner(h_low, w_low) + hh * lw * corner(h_low, w_low + 1)
            + lh * hw * corner(h_low + 1, w_low) + lh * lw * corner(h_low + 1, w_low + 1))


def modulated_deformable_im2col_pytorch(data_im, data_offset, data_mask, kernel_h, kernel_w,
                                        pad_h, pad_w, stride_h, stride_w, dilation_h,
                                        dilation_w, deformable_group):
    """Columns [C*kh*kw, B, Ho, Wo] in plain PyTorch (differentiable in all inputs)."""
    batch, channels, height, width = data_im.shape
    ho = _out_size(height, pad_h, dilation_h, kernel_h, stride_h)
    wo = _out_size(width, pad_w, dilation_w, kernel_w, stride_w)
    taps = kernel_h * kernel_w
    cpg = channels // deformable_group
    dev, dt = data_im.device, data_im.dtype
    oh = torch.arange(ho, device=dev).view(ho, 1).expand(ho, wo).reshape(-1)
    ow = torch.arange(wo, device=dev).view(1, wo).expand(ho, wo).reshape(-1)
    off = data_offset.view(batch, deformable_group, taps, 2, ho * wo)
    msk = data_mask.view(batch, deformable_group, taps, ho * wo)
    flat = data_im.reshape(batch, channels, height * width)
    cols = []
    for t in range(taps):
        i, j = divmod(t, kernel_w)
        h = (oh * stride_h - pad_h + i * dilation_h).to(dt) + off[:, :, t, 0]  # [B, dg, P]
        w = (ow * stride_w - pad_w + j * dilation_w).to(dt) + off[:, :, t, 1]
        inside = (h > -1) & (w > -1) & (h < height) & (w < width)
        hl = h.floor()
        wl = w.floor()
        lh, lw = h - hl, w - wl
        hh, hw = 1.0 - lh, 1.0 - lw
        hl, wl = hl.long(), wl.long()
        acc = 0.0
        for dy, dx, wgt in ((0, 0, hh * hw), (0, 1, hh * lw), (1, 0, lh * hw), (1, 1, lh * lw)):
            y, x = hl + dy, wl + dx
            ok = (y >= 0) & (y <= height - 1) & (x >= 0) & (x <= width - 1) & inside
            idx = (y.clamp(0, height - 1) * width + x.clamp(0, width - 1))  # [B, dg, P]
            idx = idx.repeat_interleave(cpg, dim=1)                           # [B, C, P]
            val = torch.gather(flat, 2, idx)
            acc = acc + wgt.repeat_interleave(cpg, dim=1) * val * ok.repeat_interleave(
                cpg, dim=1).to(dt)
        cols.append(acc * msk[:, :, t].repeat_interleave(cpg, dim=1))        # [B, C, P]
    col = torch.stack(cols, dim=2)                                            # [B, C, T, P]
    return col.permute(1, 2, 0, 3).reshape(channels * taps, batch, ho, wo)


def modulated_deformable_col2im_pytorch(data_col, data_im, data_offset, data_mask, kernel_h,
                                        kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h,
                                        dilation_w, deformable_group):
    """grad_im for upstream gradient data_col, by autograd through the im2col above."""
    data_im_var = data_im.detach().clone().requires_grad_(True)
    col = modulated_deformable_im2col_pytorch(data_im_var, data_offset.detach(),
                                              data_mask.detach(), kernel_h, kernel_w, pad_h,
                                              pad_w, stride_h, stride_w, dilation_h, dilation_w,
                                              deformable_group)
    return torch.autograd.grad(col, data_im_var, grad_outputs=data_col)[0]


def modulated_deformable_col2im_coord_pytorch(data_col, data_im, data_offset, data_mask,
                                              kernel_h, kernel_w, pad_h, pad_w, stride_h,
                                              stride_w, dilation_h, dilation_w,
                                              deformable_group):
    """(grad_offset, grad_mask) for upstream gradient data_col, by autograd."""
    offset_var = data_offset.detach().clone().requires_grad_(True)
    mask_var = data_mask.detach().clone().requires_grad_(True)
    col = modulated_deformable_im2col_pytorch(data_im.detach(), offset_var, mask_var, kernel_h,
                                              kernel_w, pad_h, pad_w, stride_h, stride_w,
                                              dilation_h, dilation_w, deformable_group)
    g = torch.autograd.grad(col, [offset_var, mask_var], grad_outputs=data_col)
    return g[0], g[1]


# ---------------------------------------------------------------------------------------
# Module-level operator (modulated_deform_conv.py:318-626)
# ---------------------------------------------------------------------------------------

class ModulatedDeformConv2dFunction(Function):
    """Drop-in for mmcv.ops.ModulatedDeformConv2dFunction (forward on the HIP kernels).

    groups == 1: the fused implicit-GEMM kernel builds the columns in LDS and
    multiplies them on the matrix cores; the input is viewed NHWC for it.
    groups > 1: the NCHW column kernel followed by one GEMM per group.
    """

    @staticmethod
    def forward(ctx, input, offset, mask, weight, bias=None, stride=1, padding=0, dilation=1,
                groups=1, deform_groups=1):
        if input is not None and input.dim() != 4:
            raise ValueError(f'Expected 4D tensor as input, got {input.dim()}D tensor instead.')
        ctx.stride = _pair(stride)
        ctx.padding = _pair(padding)
        ctx.dilation = _pair(dilation)
        ctx.groups = groups
        ctx.deform_groups = deform_groups
        ctx.with_bias = bias is not None
        input = input.type_as(offset)
        weight = weight.type_as(input)
        if not ctx.with_bias:
            bias = input.new_empty(0)
        ctx.save_for_backward(input, offset, mask, weight, bias)
        return _modulated_deform_conv2d_forward(input, offset, mask, weight,
                                                bias if ctx.with_bias else None, ctx.stride,
                                                ctx.padding, ctx.dilation, groups,
                                                deform_groups)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        """modulated_deform_conv.py:405-500: columns = W^T @ dO per group; grad_offset /
        grad_mask and grad_input from the column-to-image kernel; the columns of the input
        again for grad_weight = dO @ columns^T; grad_bias = sum of dO."""
        input, offset, mask, weight, bias = ctx.saved_tensors
        ext = _load_ext()
        # 16-bit inputs: the gradients are accumulated in fp32 and rounded once (the
        # reference has no 16-bit NCHW backward: its coordinate kernel is fp32/fp64 only)
        out_dtype = input.dtype
        if out_dtype in (torch.float16, torch.bfloat16):
            input, offset, mask, weight = (t.float() for t in (input, offset, mask, weight))
            grad_output = grad_output.float()
        grad_input = torch.zeros_like(input)
        grad_offset = torch.empty_like(offset)
        grad_mask = torch.empty_like(mask)
        grad_output = grad_output.contiguous()
        batch, channels, height, width = input.shape
        channels_out = weight.size(0)
        groups, deform_groups = ctx.groups, ctx.deform_groups
        c_out_g = channels_out // groups
        kernel_h, kernel_w = weight.size(2), weight.size(3)
        c_in_g_kkw = (channels // groups) * kernel_h * kernel_w
        stride_h, stride_w = ctx.stride
        pad_h, pad_w = ctx.padding
        dil_h, dil_w = ctx.dilation
        height_out = _out_size(height, pad_h, dil_h, kernel_h, stride_h)
        width_out = _out_size(width, pad_w, dil_w, kernel_w, stride_w)
        bhw = batch * height_out * width_out

        grad_out_g = grad_output.permute(1, 0, 2, 3).contiguous().view(groups, c_out_g, bhw)
        weight_g = weight.contiguous().view(groups, c_out_g, c_in_g_kkw)
        columns = input.new_empty(groups, c_in_g_kkw, bhw)
        for g in range(groups):
            torch.mm(weight_g[g].t(), grad_out_g[g], out=columns[g])
        columns = columns.view(channels * kernel_h * kernel_w, bhw)
        args = (batch, channels, height, width, height_out, width_out, kernel_h, kernel_w,
                pad_h, pad_w, stride_h, stride_w, dil_h, dil_w, deform_groups)
        ext.modulated_deformable_col2im_coord_opt_cuda(columns, input, offset, mask, *args,
                                                       grad_offset, grad_mask)
        ext.modulated_deformable_col2im_smem_cuda(columns, offset, mask, *args, grad_input)
        ext.modulated_deformable_im2col_opt_cuda(input, offset, mask, *args, columns)
        col_g = columns.view(groups, c_in_g_kkw, bhw)
        grad_weight = weight.new_empty(groups, c_out_g, c_in_g_kkw)
        for g in range(groups):
            torch.mm(grad_out_g[g], col_g[g].t(), out=grad_weight[g])
        grad_weight = grad_weight.view_as(weight)
        grad_bias = grad_output.sum(dim=(0, 2, 3)) if ctx.with_bias else None
        if out_dtype != input.dtype:
            grad_input, grad_offset, grad_mask, grad_weight = (
                t.to(out_dtype) for t in (grad_input, grad_offset, grad_mask, grad_weight))
            grad_bias = grad_bias.to(out_dtype) if grad_bias is not None else None
        return (grad_input, grad_offset, grad_mask, grad_weight, grad_bias,
                None, None, None, None, None)


def _modulated_deform_conv2d_forward(input, offset, mask, weight, bias, stride, padding,
                                     dilation, groups, deform_groups):
    ext = _load_ext()
    batch, channels, height, width = input.shape
    channels_out = weight.size(0)
    kernel_h, kernel_w = weight.size(2), weight.size(3)
    stride_h, stride_w = stride
    pad_h, pad_w = padding
    dil_h, dil_w = dilation
    ho = _out_size(height, pad_h, dil_h, kernel_h, stride_h)
    wo = _out_size(width, pad_w, dil_w, kernel_w, stride_w)
    vec = 16 // input.element_size()
    if (groups == 1 and deform_groups == 1 and input.dtype != torch.float64
            and channels % vec == 0):
        # Implicit GEMM: NHWC views of the inputs, output produced as [B, Ho, Wo, Cout].
        x_nhwc = ext.nchw_to_nhwc(input)
        off_nhwc = ext.nchw_to_nhwc(offset)
        msk_nhwc = ext.nchw_to_nhwc(mask)
        w_packed = pack_weight(weight, input.dtype)
        b = bias.to(input.dtype).contiguous() if bias is not None else None
        out = input.new_empty(batch, ho, wo, channels_out)
        ext.dcn_fused_fwd_nhwc(x_nhwc, off_nhwc, msk_nhwc, w_packed, b, batch, channels, height,
                               width, ho, wo, channels_out, kernel_h, kernel_w, pad_h, pad_w,
                               stride_h, stride_w, dil_h, dil_w, out)
        return ext.nhwc_to_nchw(out)
    # Columns [C*kh*kw, B*Ho*Wo] then one GEMM per group (modulated_deform_conv.py:369-401).
    bhw = batch * ho * wo
    columns = input.new_empty(channels * kernel_h * kernel_w, bhw)
    ext.modulated_deformable_im2col_opt_cuda(
        input.contiguous(), offset.contiguous(), mask.contiguous(), batch, channels, height,
        width, ho, wo, kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dil_h, dil_w,
        deform_groups, columns)
    c_out_g = channels_out // groups
    c_in_g_kkw = (channels // groups) * kernel_h * kernel_w
    col_g = columns.view(groups, c_in_g_kkw, bhw)
    weight_g = weight.contiguous().view(groups, c_out_g, c_in_g_kkw)
    if groups == 1:
        output_flat = torch.mm(weight_g[0], col_g[0]).unsqueeze(0)
    else:
        output_flat = torch.empty(groups, c_out_g, bhw, dtype=columns.dtype,
                                  device=columns.device)
        for g in range(groups):
            torch.mm(weight_g[g], col_g[g], out=output_flat[g])
    output = output_flat.view(channels_out, batch, ho, wo).permute(1, 0, 2, 3).contiguous()
    if bias is not None:
        output = output + bias.view(1, -1, 1, 1)
    return output


modulated_deform_conv2d = ModulatedDeformConv2dFunction.apply


class ModulatedDeformConv2d(nn.Module):
    """Drop-in replacement for mmcv.ops.ModulatedDeformConv2d."""

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, dilation=1,
                 groups=1, deform_groups=1, bias=True):
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = _pair(kernel_size)
        self.stride = _pair(stride)
        self.padding = _pair(padding)
        self.dilation = _pair(dilation)
        self.groups = groups
        self.deform_groups = deform_groups
        self.transposed = False
        self.output_padding = _single(0)
        self.weight = nn.Parameter(
            torch.empty(out_channels, in_channels // groups, *self.kernel_size))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_channels))
        else:
            self.register_parameter('bias', None)
        self.init_weights()

    def init_weights(self):
        n = self.in_channels
        for k in self.kernel_size:
            n *= k
        stdv = 1. / math.sqrt(n)
        self.weight.data.uniform_(-stdv, stdv)
        if self.bias is not None:
            self.bias.data.zero_()

    def forward(self, x, offset, mask):
        return modulated_deform_conv2d(x, offset, mask, self.weight, self.bias, self.stride,
                                       self.padding, self.dilation, self.groups,
                                       self.deform_groups)


class ModulatedDeformConv2dPack(ModulatedDeformConv2d):
    """DCNv2 with its own offset/mask conv; drop-in for mmcv.ops.ModulatedDeformConv2dPack
    and loads mmcv checkpoints (including the v1 ``_offset`` key names).

    backend (kwarg, else env DCN_BACKEND, default 'fuse_c'):
      'fuse_c'   NHWC path of dcn_split_nhwc (offset conv + fused gather/GEMM kernel),
      'tilelang' NHWC path of fused_tl (same kernels on this build),
      'cuda'     NCHW path of modulated_deform_conv2d.
    'fuse_c' / 'tilelang' need groups == 1 and deform_groups == 1, else 'cuda' is used.
    """

    _version = 2

    def __init__(self, *args, **kwargs):
        self.backend = kwargs.pop('backend', os.environ.get('DCN_BACKEND', 'fuse_c'))
        super().__init__(*args, **kwargs)
        self.conv_offset = nn.Conv2d(
            self.in_channels,
            self.deform_groups * 3 * self.kernel_size[0] * self.kernel_size[1],
            kernel_size=self.kernel_size,
            stride=self.stride,
            padding=self.padding,
            dilation=self.dilation,
            bias=True)
        self.init_weights()

    def init_weights(self):
        super().init_weights()
        if hasattr(self, 'conv_offset'):
            self.conv_offset.weight.data.zero_()
            self.conv_offset.bias.data.zero_()

    def forward(self, x):
        backend = getattr(self, 'backend', 'fuse_c')
        if backend in ('fuse_c', 'tilelang') and (self.groups != 1 or self.deform_groups != 1):
            backend = 'cuda'
        if backend == 'tilelang':
            from .fused_tl import dcn_apply_nchw
            return dcn_apply_nchw(x, self.conv_offset.weight, self.conv_offset.bias,
                                  self.weight, self.bias, self.stride, self.padding,
                                  self.dilation)
        if backend == 'fuse_c':
            from .dcn_split_nhwc import dcn_apply_nchw as dcn_apply_nchw_fusec
            return dcn_apply_nchw_fusec(x, self.conv_offset.weight, self.conv_offset.bias,
                                        self.weight, self.bias, self.stride, self.padding,
                                        self.dilation)
        out = self.conv_offset(x)
        o1, o2, mask = torch.chunk(out, 3, dim=1)
        offset = torch.cat((o1, o2), dim=1)
        mask = torch.sigmoid(mask)
        if os.environ.get("ENABLE_CHANNEL_LAST", "false").lower() in ("1", "true", "yes", "on"):
            x = x.to(memory_format=torch.contiguous_format)
            offset = offset.to(memory_format=torch.contiguous_format)
            mask = mask.to(memory_format=torch.contiguous_format)
            return modulated_deform_conv2d(
                x, offset, mask, self.weight.to(memory_format=torch.contiguous_format),
                self.bias, self.stride, self.padding, self.dilation, self.groups,
                self.deform_groups).to(memory_format=torch.channels_last)
        return modulated_deform_conv2d(x, offset, mask, self.weight, self.bias, self.stride,
                                       self.padding, self.dilation, self.groups,
                                       self.deform_groups)

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        version = local_metadata.get('version', None)
        if version is None or version < 2:
            # mmcv v1 named the offset conv `<name>_offset`.
            for suffix in ('weight', 'bias'):
                new_key = prefix + 'conv_offset.' + suffix
                old_key = prefix[:-1] + '_offset.' + suffix
                if new_key not in state_dict and old_key in state_dict:
                    state_dict[new_key] = state_dict.pop(old_key)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)
