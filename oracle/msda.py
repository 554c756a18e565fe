"""MSDA forward and backward restated on the CPU (test oracle; see oracle/__init__.py).

Reference (naotic/bev-kernels csrc_musa/msda/):
  bilinear with per-corner zeroing      ms_deform_attn_kernels.cuh:7-49
  loc/attn indexing (loc[...,0] = x/w)  ms_deform_attn_kernels.cuh:104-113
  level base lsi[l] * heads * D         ms_deform_attn_kernels.cuh:116-132
  h = loc_y*H - 0.5, gate, accumulate   ms_deform_attn_kernels.cuh:252-259 (l-major, then p)
  output index / zero init              ms_deform_attn_kernels.cuh:281-283, binding_musa.mu:311-312
  backward per sample, channel sums     ms_deform_attn_kernels.cuh:427-490, :763-770
The reference has no PyTorch golden for MSDA; these are its kernel semantics. Pins:
forward against brute_force and the F.grid_sample closed form; backward against
autograd of both forward restatements and finite differences (tests/test_oracle_msda.py).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def _coords(loc_h, loc_w, H, W, coord_dtype):
    """h_im = loc_y * H - 0.5, w_im = loc_x * W - 0.5 (ms_deform_attn_kernels.cuh:252-253,
    :714-715). The reference declares them `float`: coord_dtype=torch.float32 rounds the
    exact value once to fp32, as an fp32 kernel computing them with one fused
    multiply-add does; None keeps them exact."""
    h_im = loc_h * H - 0.5
    w_im = loc_w * W - 0.5
    if coord_dtype is not None:
        h_im = h_im.to(coord_dtype).to(loc_h.dtype)
        w_im = w_im.to(coord_dtype).to(loc_w.dtype)
    return h_im, w_im


def forward(value, spatial_shapes, level_start_index, sampling_loc, attn_weight,
            coord_dtype=None):
    """Direct restatement: out[b,q,h*D+c] = sum_l sum_p attn * bilinear. Loops over
    (l, p) like the kernels, vectorised over (b, q, head, c)."""
    B, S, NH, D = value.shape
    _, Lq, _, L, P, _ = sampling_loc.shape
    dt = value.dtype
    out = torch.zeros(B, Lq, NH, D, dtype=dt)
    b_idx = torch.arange(B).view(B, 1, 1)
    h_idx = torch.arange(NH).view(1, 1, NH)
    shapes = spatial_shapes.tolist()
    starts = level_start_index.tolist()
    for l in range(L):
        H, W = int(shapes[l][0]), int(shapes[l][1])
        start = int(starts[l])
        for p in range(P):
            loc_w = sampling_loc[:, :, :, l, p, 0]                 # [B, Lq, NH]
            loc_h = sampling_loc[:, :, :, l, p, 1]
            wgt = attn_weight[:, :, :, l, p]
            h_im, w_im = _coords(loc_h, loc_w, H, W, coord_dtype)
            inside = (h_im > -1) & (w_im > -1) & (h_im < H) & (w_im < W)
            h_low = torch.floor(h_im)
            w_low = torch.floor(w_im)
            lh = h_im - h_low
            lw = w_im - w_low
            hh = 1 - lh
            hw = 1 - lw
            h_low = h_low.long()
            w_low = w_low.long()

            def corner(iy, ix):
                ok = (iy >= 0) & (iy <= H - 1) & (ix >= 0) & (ix <= W - 1) & inside
                pos = start + iy.clamp(0, H - 1) * W + ix.clamp(0, W - 1)
                v = value[b_idx, pos, h_idx]                       # [B, Lq, NH, D]
                return torch.where(ok.unsqueeze(-1), v, torch.zeros_like(v))

            v1 = corner(h_low, w_low)
            v2 = corner(h_low, w_low + 1)
            v3 = corner(h_low + 1, w_low)
            v4 = corner(h_low + 1, w_low + 1)
            val = ((hh * hw).unsqueeze(-1) * v1 + (hh * lw).unsqueeze(-1) * v2
                   + (lh * hw).unsqueeze(-1) * v3 + (lh * lw).unsqueeze(-1) * v4)
            contrib = val * wgt.unsqueeze(-1)
            out += torch.where(inside.unsqueeze(-1), contrib, torch.zeros_like(contrib))
    return out.reshape(B, Lq, NH * D)


def forward_grid_sample(value, spatial_shapes, level_start_index, sampling_loc, attn_weight):
    """Closed form through F.grid_sample(align_corners=False, padding_mode='zeros'):
    grid g = 2*loc - 1 maps to ((g+1)*H - 1)/2 = loc*H - 0.5, and zero padding is the
    per-corner zeroing (the outer gate only drops samples whose corners are all out)."""
    B, S, NH, D = value.shape
    _, Lq, _, L, P, _ = sampling_loc.shape
    out = None
    shapes = spatial_shapes.tolist()
    starts = level_start_index.tolist()
    for l in range(L):
        H, W = int(shapes[l][0]), int(shapes[l][1])
        start = int(starts[l])
        v = value[:, start:start + H * W].permute(0, 2, 3, 1).reshape(B * NH, D, H, W)
        grid = 2 * sampling_loc[:, :, :, l] - 1                    # [B, Lq, NH, P, 2]
        grid = grid.permute(0, 2, 1, 3, 4).reshape(B * NH, Lq, P, 2)
        samp = F.grid_sample(v, grid, mode="bilinear", padding_mode="zeros",
                             align_corners=False)                 # [B*NH, D, Lq, P]
        w = attn_weight[:, :, :, l].permute(0, 2, 1, 3).reshape(B * NH, 1, Lq, P)
        term = (samp * w).sum(-1)                                  # [B*NH, D, Lq]
        out = term if out is None else out + term
    if out is None:
        return torch.zeros(B, Lq, NH * D, dtype=value.dtype)
    return out.view(B, NH, D, Lq).permute(0, 3, 1, 2).reshape(B, Lq, NH * D)


def brute_force(value, spatial_shapes, level_start_index, sampling_loc, attn_weight):
    """Scalar loops over every (b, q, head, c, l, p), Python floats; tiny shapes only."""
    B, S, NH, D = value.shape
    _, Lq, _, L, P, _ = sampling_loc.shape
    vs = value.double().tolist()
    ls = sampling_loc.double().tolist()
    ws = attn_weight.double().tolist()
    shapes = spatial_shapes.tolist()
    starts = level_start_index.tolist()
    out = torch.zeros(B, Lq, NH * D, dtype=torch.float64)
    for b in range(B):
        for q in range(Lq):
            for h in range(NH):
                for c in range(D):
                    acc = 0.0
                    for l in range(L):
                        H, W = shapes[l]
                        for p in range(P):
                            x, y = ls[b][q][h][l][p]
                            hi = y * H - 0.5
                            wi = x * W - 0.5
                            if not (-1 < hi < H and -1 < wi < W):
                                continue
                            y0, x0 = math.floor(hi), math.floor(wi)
                            ly, lx = hi - y0, wi - x0
                            s = 0.0
                            for yy, xx, f in ((y0, x0, (1 - ly) * (1 - lx)),
                                              (y0, x0 + 1, (1 - ly) * lx),
                                              (y0 + 1, x0, ly * (1 - lx)),
                                              (y0 + 1, x0 + 1, ly * lx)):
                                if 0 <= yy < H and 0 <= xx < W:
                                    s += f * vs[b][starts[l] + yy * W + xx][h][c]
                            acc += s * ws[b][q][h][l][p]
                    out[b, q, h * D + c] = acc
    return out


def backward(value, spatial_shapes, level_start_index, sampling_loc, attn_weight, grad_output,
             coord_dtype=None):
    """MSDA backward restated from the reference's per-sample gradient
    (ms_deform_attn_kernels.cuh:427-490, reduced over channels as :763-770):
      grad_value[corner] += w_corner * top * a            (only corners inside the level)
      grad_loc_x = W * sum_c top * a * (-hh*v1 + hh*v2 - lh*v3 + lh*v4)
      grad_loc_y = H * sum_c top * a * (-hw*v1 - lw*v2 + hw*v3 + lw*v4)
      grad_attn  = sum_c top * (w1*v1 + w2*v2 + w3*v3 + w4*v4)
    with all three zero for a sample outside (-1, H) x (-1, W). coord_dtype as forward.
    grad_output [B, Lq, NH*D] -> (grad_value, grad_sampling_loc, grad_attn_weight)."""
    B, S, NH, D = value.shape
    _, Lq, _, L, P, _ = sampling_loc.shape
    dt = value.dtype
    top = grad_output.reshape(B, Lq, NH, D).to(dt)
    g_value = torch.zeros_like(value)
    g_loc = torch.zeros_like(sampling_loc)
    g_attn = torch.zeros_like(attn_weight)
    b_idx = torch.arange(B).view(B, 1, 1).expand(B, Lq, NH)
    h_idx = torch.arange(NH).view(1, 1, NH).expand(B, Lq, NH)
    shapes = spatial_shapes.tolist()
    starts = level_start_index.tolist()
    flat = g_value.view(B * S * NH, D)
    for l in range(L):
        H, W = int(shapes[l][0]), int(shapes[l][1])
        start = int(starts[l])
        for p in range(P):
            loc_w = sampling_loc[:, :, :, l, p, 0]
            loc_h = sampling_loc[:, :, :, l, p, 1]
            a = attn_weight[:, :, :, l, p]
            h_im, w_im = _coords(loc_h, loc_w, H, W, coord_dtype)
            inside = (h_im > -1) & (w_im > -1) & (h_im < H) & (w_im < W)
            h_low = torch.floor(h_im)
            w_low = torch.floor(w_im)
            lh = h_im - h_low
            lw = w_im - w_low
            hh = 1 - lh
            hw = 1 - lw
            h_low = h_low.long()
            w_low = w_low.long()
            ta = top * a.unsqueeze(-1)                                  # [B, Lq, NH, D]
            vs = []
            for iy, ix, wgt in ((h_low, w_low, hh * hw), (h_low, w_low + 1, hh * lw),
                                (h_low + 1, w_low, lh * hw), (h_low + 1, w_low + 1, lh * lw)):
                ok = (iy >= 0) & (iy <= H - 1) & (ix >= 0) & (ix <= W - 1) & inside
                pos = start + iy.clamp(0, H - 1) * W + ix.clamp(0, W - 1)
                v = value[b_idx, pos, h_idx]
                v = torch.where(ok.unsqueeze(-1), v, torch.zeros_like(v))
                vs.append(v)
                row = ((b_idx * S + pos) * NH + h_idx)[ok]
                flat.index_add_(0, row, (wgt.unsqueeze(-1) * ta)[ok])
            v1, v2, v3, v4 = vs
            zero = torch.zeros_like(lh)
            gx = W * (ta * (-hh.unsqueeze(-1) * v1 + hh.unsqueeze(-1) * v2
                            - lh.unsqueeze(-1) * v3 + lh.unsqueeze(-1) * v4)).sum(-1)
            gy = H * (ta * (-hw.unsqueeze(-1) * v1 - lw.unsqueeze(-1) * v2
                            + hw.unsqueeze(-1) * v3 + lw.unsqueeze(-1) * v4)).sum(-1)
            ga = (top * ((hh * hw).unsqueeze(-1) * v1 + (hh * lw).unsqueeze(-1) * v2
                         + (lh * hw).unsqueeze(-1) * v3 + (lh * lw).unsqueeze(-1) * v4)).sum(-1)
            g_loc[:, :, :, l, p, 0] = torch.where(inside, gx, zero)
            g_loc[:, :, :, l, p, 1] = torch.where(inside, gy, zero)
            g_attn[:, :, :, l, p] = torch.where(inside, ga, zero)
    return g_value, g_loc, g_attn
