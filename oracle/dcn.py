"""DCNv2 forward restated on the CPU (test oracle; see oracle/__init__.py).

All functions compute in the dtype of their inputs; the tests pass float64 copies of the
(possibly fp16/bf16-rounded) kernel inputs so the oracle itself adds no rounding that
matters at the 1e-4 tolerance.

Reference (naotic/bev-kernels):
  _bilinear_sample                modulated_deform_conv.py:184-213
  modulated_deformable_im2col     modulated_deform_conv.py:216-266
  ModulatedDeformConv2dFunction   modulated_deform_conv.py:331-403 (forward composition)
  _bilinear_nhwc                  fused_tl.py:146-174
  dcn_columns_golden_nhwc         fused_tl.py:177-201
  dcn_forward_golden_nhwc         fused_tl.py:204-227
  Pack offset/mask split          modulated_deform_conv.py:610-613, dcn_split_nhwc.py:131-132
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def out_size(size, pad, dil, k, stride):
    """modulated_deform_conv.py:364-365."""
    return (size + 2 * pad - (dil * (k - 1) + 1)) // stride + 1


def bilinear_plane(plane, h, w):
    """Bilinear sample of plane [..., H, W] (leading dims broadcast against h, w's
    leading dims) at float coordinates; a neighbour outside [0,H-1]x[0,W-1] counts as 0.
    modulated_deform_conv.py:184-213 (corner order v1..v4, weights hh*hw, hh*lw, lh*hw,
    lh*lw, summed left to right)."""
    H, W = plane.shape[-2:]
    h_low = torch.floor(h)
    w_low = torch.floor(w)
    lh = h - h_low
    lw = w - w_low
    hh = 1.0 - lh
    hw = 1.0 - lw
    h_low = h_low.long()
    w_low = w_low.long()
    flat = plane.reshape(*plane.shape[:-2], H * W)

    def get(iy, ix):
        valid = (iy >= 0) & (iy <= H - 1) & (ix >= 0) & (ix <= W - 1)
        idx = iy.clamp(0, H - 1) * W + ix.clamp(0, W - 1)
        val = torch.gather(flat, -1, idx)
        return torch.where(valid, val, torch.zeros_like(val))

    v1 = get(h_low, w_low)
    v2 = get(h_low, w_low + 1)
    v3 = get(h_low + 1, w_low)
    v4 = get(h_low + 1, w_low + 1)
    return hh * hw * v1 + hh * lw * v2 + lh * hw * v3 + lh * lw * v4


def im2col_nchw(data_im, data_offset, data_mask, kernel_h, kernel_w, pad_h, pad_w, stride_h,
                stride_w, dilation_h, dilation_w, deformable_group):
    """Columns [C*kh*kw, B, Ho, Wo], row c*kh*kw + i*kw + j.
    modulated_deform_conv.py:216-266. The reference loops over (c, i, j, b) and samples
    one plane per iteration; here the loop is over (i, j) and all (b, c) planes are
    sampled at once, with the same per-element arithmetic."""
    B, C, H, W = data_im.shape
    Ho = out_size(H, pad_h, dilation_h, kernel_h, stride_h)
    Wo = out_size(W, pad_w, dilation_w, kernel_w, stride_w)
    T = kernel_h * kernel_w
    cpg = C // deformable_group
    dt = data_im.dtype
    h_grid = torch.arange(Ho, dtype=dt).view(Ho, 1).expand(Ho, Wo).reshape(-1)
    w_grid = torch.arange(Wo, dtype=dt).view(1, Wo).expand(Ho, Wo).reshape(-1)
    dg_of_c = torch.arange(C) // cpg                                      # [C]
    cols = torch.empty(C, T, B, Ho * Wo, dtype=dt)
    for i in range(kernel_h):
        for j in range(kernel_w):
            t = i * kernel_w + j
            # offsets/mask of channel c come from its deformable group (:249-251)
            off = data_offset.view(B, deformable_group, 2 * T, Ho * Wo)
            offset_h = off[:, dg_of_c, 2 * t]                             # [B, C, P]
            offset_w = off[:, dg_of_c, 2 * t + 1]
            mask_val = data_mask.view(B, deformable_group, T, Ho * Wo)[:, dg_of_c, t]
            h_in = h_grid * stride_h - pad_h
            w_in = w_grid * stride_w - pad_w
            h_im = h_in + i * dilation_h + offset_h
            w_im = w_in + j * dilation_w + offset_w
            valid = (h_im > -1) & (w_im > -1) & (h_im < H) & (w_im < W)   # :256
            h_im_c = torch.where(valid, h_im, torch.zeros_like(h_im))
            w_im_c = torch.where(valid, w_im, torch.zeros_like(w_im))
            val = bilinear_plane(data_im, h_im_c, w_im_c)                 # [B, C, P]
            val = torch.where(valid, val, torch.zeros_like(val))
            cols[:, t] = (val * mask_val).permute(1, 0, 2)
    return cols.reshape(C * T, B, Ho, Wo)


def _round_cols(cols, col_dtype):
    """Columns rounded to the kernel's storage dtype, as the reference stores them: its
    column buffer is allocated in the input dtype (modulated_deform_conv.py:370,
    dcn_split_nhwc.py:40) and the fused kernel's A tile is `dtype` (fused_tl.py:68). The
    GEMM after it stays in the oracle's precision."""
    if col_dtype is None:
        return cols
    return cols.to(col_dtype).to(cols.dtype)


def forward_nchw(x, offset, mask, weight, bias=None, stride=(1, 1), padding=(0, 0),
                 dilation=(1, 1), groups=1, deform_groups=1, col_dtype=None):
    """ModulatedDeformConv2dFunction.forward, modulated_deform_conv.py:331-403:
    columns, one GEMM per group, [Cout, B, Ho, Wo] -> [B, Cout, Ho, Wo], + bias.
    col_dtype: round the columns to this dtype first (see _round_cols)."""
    B, C, H, W = x.shape
    Cout, _, kh, kw = weight.shape
    (sh, sw), (ph, pw), (dh, dw) = stride, padding, dilation
    Ho = out_size(H, ph, dh, kh, sh)
    Wo = out_size(W, pw, dw, kw, sw)
    cols = _round_cols(im2col_nchw(x, offset, mask, kh, kw, ph, pw, sh, sw, dh, dw,
                                   deform_groups), col_dtype)
    bhw = B * Ho * Wo
    cin_g_kk = (C // groups) * kh * kw
    col_g = cols.reshape(groups, cin_g_kk, bhw)
    w_g = weight.reshape(groups, Cout // groups, cin_g_kk)
    out = torch.bmm(w_g, col_g).reshape(Cout, B, Ho, Wo).permute(1, 0, 2, 3)
    if bias is not None:
        out = out + bias.view(1, -1, 1, 1)
    return out.contiguous()


def bilinear_nhwc(im_b, h, w, gate=True):
    """fused_tl.py:146-174: im_b [H, W, C]; h, w [P] -> [P, C] with per-corner zeroing
    and the outer gate -1 < h < H, -1 < w < W. gate=False drops the outer gate and keeps
    only the per-corner checks, as the reference's NHWC kernels do
    (dcn_fused_nhwc_kernel.cuh:270-301, :642-711): the same values for finite coordinates,
    but at h = -1 (or w = -1) the derivative is the one-sided one of the cell [-1, 0]
    instead of 0."""
    H, W, C = im_b.shape
    h_low = torch.floor(h)
    w_low = torch.floor(w)
    lh = h - h_low
    lw = w - w_low
    hh = 1.0 - lh
    hw = 1.0 - lw
    h_low = h_low.long()
    w_low = w_low.long()

    def corner(iy, ix):
        valid = (iy >= 0) & (iy <= H - 1) & (ix >= 0) & (ix <= W - 1)
        val = im_b[iy.clamp(0, H - 1), ix.clamp(0, W - 1)]
        return torch.where(valid.unsqueeze(-1), val, torch.zeros_like(val))

    out = ((hh * hw).unsqueeze(-1) * corner(h_low, w_low)
           + (hh * lw).unsqueeze(-1) * corner(h_low, w_low + 1)
           + (lh * hw).unsqueeze(-1) * corner(h_low + 1, w_low)
           + (lh * lw).unsqueeze(-1) * corner(h_low + 1, w_low + 1))
    if not gate:
        return out
    outer = (h > -1) & (w > -1) & (h < H) & (w < W)
    return torch.where(outer.unsqueeze(-1), out, torch.zeros_like(out))


def columns_nhwc(x, offset, mask, kh, kw, sh, sw, ph, pw, dh, dw, gate=True,
                 coord_dtype=None):
    """fused_tl.py:177-201: columns [B*Ho*Wo, T*C], k = t*C + c (gate: see bilinear_nhwc).

    coord_dtype=torch.float32 rounds each sampling coordinate (integer tap position +
    offset) once to fp32 and evaluates everything else in x's dtype: the reference's
    kernels hold the coordinate in a float (dcn_fused_nhwc_kernel.cuh:140-141,
    fused_tl.py:114-115), and an fp16 / fp32 offset added to a tap position can need more
    than 24 significant bits (39 - 0.00173 needs 26). The rounding is an identity for
    autograd, so gradients are those at the rounded coordinate."""
    B, H, W, C = x.shape
    T = kh * kw
    Ho = out_size(H, ph, dh, kh, sh)
    Wo = out_size(W, pw, dw, kw, sw)
    dt = x.dtype
    oh = torch.arange(Ho, dtype=dt).view(Ho, 1).expand(Ho, Wo).reshape(-1)
    ow = torch.arange(Wo, dtype=dt).view(1, Wo).expand(Ho, Wo).reshape(-1)
    cols = torch.zeros(B, Ho * Wo, T, C, dtype=dt)
    for b in range(B):
        for t in range(T):
            ki, kj = t // kw, t % kw
            h_im = oh * sh - ph + ki * dh + offset[b, :, :, 2 * t].reshape(-1)
            w_im = ow * sw - pw + kj * dw + offset[b, :, :, 2 * t + 1].reshape(-1)
            if coord_dtype is not None:
                h_im = h_im + (h_im.detach().to(coord_dtype).to(dt) - h_im.detach())
                w_im = w_im + (w_im.detach().to(coord_dtype).to(dt) - w_im.detach())
            samp = bilinear_nhwc(x[b], h_im, w_im, gate)
            cols[b, :, t, :] = samp * mask[b, :, :, t].reshape(-1, 1)
    return cols.reshape(B * Ho * Wo, T * C)


def forward_nhwc(x, offset, mask, weight, bias=None, stride=1, padding=0, dilation=1,
                 col_dtype=None, gate=True, coord_dtype=None):
    """fused_tl.py:204-227: cols @ weight.permute(2,3,1,0).reshape(K, Cout) (+ bias).
    col_dtype: round the columns to this dtype first (see _round_cols); gate: see
    bilinear_nhwc; coord_dtype: see columns_nhwc."""
    def two(v):
        return (v, v) if isinstance(v, int) else tuple(v)
    (sh, sw), (ph, pw), (dh, dw) = two(stride), two(padding), two(dilation)
    B, H, W, C = x.shape
    Cout, _, kh, kw = weight.shape
    Ho = out_size(H, ph, dh, kh, sh)
    Wo = out_size(W, pw, dw, kw, sw)
    cols = _round_cols(columns_nhwc(x, offset, mask, kh, kw, sh, sw, ph, pw, dh, dw, gate,
                                    coord_dtype), col_dtype)
    out = (cols @ weight.permute(2, 3, 1, 0).reshape(kh * kw * C, Cout)).view(B, Ho, Wo, Cout)
    if bias is not None:
        out = out + bias.view(1, 1, 1, -1)
    return out


def fused_front_end_columns(x, w_off_tc, b_off, kh, kw, stride=1, padding=0, dilation=1,
                            col_dtype=None):
    """Fused NHWC front end (K12, dcn_fused_nhwc_kernel.cuh:211-303): y = conv(x, w_off) +
    b_off with the deformable taps' stride / padding / dilation (:236-258), offsets =
    y[..., :2T] ((dy, dx) per tap, :266-267), mask = sigmoid(y[..., 2T:3T]) (:268), then the
    NHWC columns (:270-301). x [B, H, W, C]; w_off_tc [3T, T, C] (= [3T, C, kh, kw]
    permuted (0, 2, 3, 1)); b_off [3T]."""
    def two(v):
        return (v, v) if isinstance(v, int) else tuple(v)
    (sh, sw), (ph, pw), (dh, dw) = two(stride), two(padding), two(dilation)
    T = kh * kw
    C = x.shape[-1]
    w_nchw = w_off_tc.reshape(3 * T, kh, kw, C).permute(0, 3, 1, 2)
    y = F.conv2d(x.permute(0, 3, 1, 2), w_nchw, b_off, (sh, sw), (ph, pw), (dh, dw))
    off, mask = split_y_nhwc(y.permute(0, 2, 3, 1), T)
    cols = columns_nhwc(x, off, mask, kh, kw, sh, sw, ph, pw, dh, dw)
    return _round_cols(cols, col_dtype)


def offset_conv_nhwc(x, w_off, b_off=None, stride=1, padding=0, dilation=1):
    """Offset conv of the NHWC front end (fused_tl.py:419-470, dcn_split_nhwc.py:168-172):
    y [B, Ho, Wo, 3T] = conv(x, w_off) + b_off, x [B, H, W, C], w_off [3T, C, kh, kw] (the
    library convolution in the caller's precision: float64 here)."""
    def two(v):
        return (v, v) if isinstance(v, int) else tuple(v)
    y = F.conv2d(x.permute(0, 3, 1, 2), w_off, b_off, two(stride), two(padding), two(dilation))
    return y.permute(0, 2, 3, 1)


def mega_forward_nhwc(x, w_off, b_off, weight, bias=None, stride=1, padding=0, dilation=1,
                      col_dtype=None, relu=False):
    """Whole NHWC forward with the offset conv inside (fused_tl.py:565-766): y =
    offset_conv_nhwc, offsets y[..., :2T], mask sigmoid(y[..., 2T:]) (split_y_nhwc), then
    forward_nhwc; relu: the ReLU epilogue of dcn_split_nhwc.py:190-196."""
    kh, kw = weight.shape[2], weight.shape[3]
    y = offset_conv_nhwc(x, w_off, b_off, stride, padding, dilation)
    off, mask = split_y_nhwc(y, kh * kw)
    out = forward_nhwc(x, off, mask, weight, bias, stride, padding, dilation,
                       col_dtype=col_dtype)
    return torch.relu(out) if relu else out


def split_y_nhwc(y, taps):
    """Raw offset-conv output y [..., 3T] -> (offset y[..., :2T], mask sigmoid(y[..., 2T:]))
    (dcn_split_nhwc.py:131-132; dcn_fused_nhwc_kernel.cuh:126-131)."""
    return y[..., :2 * taps], torch.sigmoid(y[..., 2 * taps:])


def split_y_nchw(y, taps):
    """Pack module: chunk(3) -> offset cat(o1, o2), mask sigmoid(o3)
    (modulated_deform_conv.py:610-613)."""
    o1, o2, m = torch.chunk(y, 3, dim=1)
    return torch.cat((o1, o2), dim=1), torch.sigmoid(m)


def brute_force_nchw(x, offset, mask, weight, bias, stride, padding, dilation, deform_groups=1):
    """Scalar loops over (b, co, oh, ow, ci, i, j): the DCNv2 definition, for tiny shapes.
    Independent of the vectorised code above (Python floats, float64)."""
    B, C, H, W = x.shape
    Cout, Cg, kh, kw = weight.shape
    groups = C // Cg
    (sh, sw), (ph, pw), (dh, dw) = stride, padding, dilation
    Ho = out_size(H, ph, dh, kh, sh)
    Wo = out_size(W, pw, dw, kw, sw)
    cpg = C // deform_groups
    xs = x.double().tolist()
    os_ = offset.double().tolist()
    ms = mask.double().tolist()
    ws = weight.double().tolist()
    out = [[[[0.0] * Wo for _ in range(Ho)] for _ in range(Cout)] for _ in range(B)]

    def px(b, c, y, xx):
        if 0 <= y < H and 0 <= xx < W:
            return xs[b][c][y][xx]
        return 0.0

    for b in range(B):
        for oh in range(Ho):
            for ow in range(Wo):
                taps = {}
                for c in range(C):
                    g = c // cpg
                    for i in range(kh):
                        for j in range(kw):
                            t = i * kw + j
                            dy = os_[b][g * 2 * kh * kw + 2 * t][oh][ow]
                            dx = os_[b][g * 2 * kh * kw + 2 * t + 1][oh][ow]
                            m = ms[b][g * kh * kw + t][oh][ow]
                            h = oh * sh - ph + i * dh + dy
                            w = ow * sw - pw + j * dw + dx
                            v = 0.0
                            if -1 < h < H and -1 < w < W:
                                y0, x0 = math.floor(h), math.floor(w)
                                ly, lx = h - y0, w - x0
                                v = ((1 - ly) * (1 - lx) * px(b, c, y0, x0)
                                     + (1 - ly) * lx * px(b, c, y0, x0 + 1)
                                     + ly * (1 - lx) * px(b, c, y0 + 1, x0)
                                     + ly * lx * px(b, c, y0 + 1, x0 + 1))
                            taps[(c, i, j)] = v * m
                for co in range(Cout):
                    g = co // (Cout // groups)
                    s = 0.0
                    for cl in range(Cg):
                        c = g * Cg + cl
                        for i in range(kh):
                            for j in range(kw):
                                s += ws[co][cl][i][j] * taps[(c, i, j)]
                    if bias is not None:
                        s += float(bias[co])
                    out[b][co][oh][ow] = s
    return torch.tensor(out, dtype=torch.float64)
