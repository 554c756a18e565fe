"""Seeded synthetic inputs for the BASELINE configurations (test / bench infrastructure).

Every tensor is drawn on the CPU from one torch.Generator in the order listed, so the
oracle and the kernels see identical values. `scale_q` (MSDA) and `batch` (DCN) shrink a
configuration for quick tests while keeping its distributions and geometry.
"""
from __future__ import annotations

import torch

# ---------------------------------------------------------------------------------------
# DCNv2
# ---------------------------------------------------------------------------------------

DCN_CONFIGS = {
    # name: (seed, batch, Cin, Cout, H, W, offset_std)
    "dcn_c1": (0, 1, 64, 64, 32, 32, 1.5),      # CPU golden config, fp32 NCHW
    "dcn_res4": (1, 6, 256, 256, 58, 100, 2.0),  # ResNet-101-DCN res4, 6 cameras
    "dcn_res5": (2, 6, 512, 512, 29, 50, 2.0),   # ResNet-101-DCN res5, 6 cameras
}


def dcn_inputs(name: str, batch: int | None = None, seed: int | None = None):
    """NCHW fp32 inputs: x ~ N(0,1), offset ~ N(0, std^2) px [B, 18, H, W] with the
    (dy, dx) interleave, mask = sigmoid(N(0,1)) [B, 9, H, W], weight Kaiming-normal
    [Cout, Cin, 3, 3], bias = 0. 3x3, stride 1, pad 1, dil 1, dg 1."""
    s, b, cin, cout, h, w, std = DCN_CONFIGS[name]
    b = b if batch is None else batch
    g = torch.Generator().manual_seed(s if seed is None else seed)
    x = torch.randn(b, cin, h, w, generator=g)
    offset = std * torch.randn(b, 18, h, w, generator=g)
    mask = torch.sigmoid(torch.randn(b, 9, h, w, generator=g))
    weight = torch.empty(cout, cin, 3, 3)
    torch.nn.init.kaiming_normal_(weight, generator=g)
    bias = torch.zeros(cout)
    return dict(x=x, offset=offset, mask=mask, weight=weight, bias=bias, stride=(1, 1),
                padding=(1, 1), dilation=(1, 1))


def round_to(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Round to `dtype` and come back to float64 (the exact values the kernel sees)."""
    return t.to(dtype).to(torch.float64)


def nchw_to_nhwc(d):
    """NHWC views of a dcn_inputs dict: x [B,H,W,C], offset [B,Ho,Wo,2T] (interleave
    kept), mask [B,Ho,Wo,T]."""
    return dict(d, x=d["x"].permute(0, 2, 3, 1).contiguous(),
                offset=d["offset"].permute(0, 2, 3, 1).contiguous(),
                mask=d["mask"].permute(0, 2, 3, 1).contiguous())


# ---------------------------------------------------------------------------------------
# MSDA (BASELINE configs[2..4])
# ---------------------------------------------------------------------------------------

MSDA_CONFIGS = {
    # name: (seed, batch, shapes, num_query, heads, head_dim, points)
    "msda_detr": (3, 2, [(100, 150), (50, 75), (25, 38), (13, 19)], 19947, 8, 32, 4),
    "msda_tsa": (4, 2, [(200, 200)], 40000, 8, 32, 4),
    "msda_sca": (5, 6, [(116, 200), (58, 100), (29, 50), (15, 25)], 10000, 8, 32, 8),
}


def msda_meta(shapes):
    spatial_shapes = torch.tensor(shapes, dtype=torch.int64)
    areas = spatial_shapes[:, 0] * spatial_shapes[:, 1]
    level_start_index = torch.cat([torch.zeros(1, dtype=torch.int64), areas.cumsum(0)[:-1]])
    return spatial_shapes, level_start_index, int(areas.sum())


def msda_inputs(name: str, scale_q: float = 1.0, batch: int | None = None):
    """fp32 inputs of one MSDA configuration.

    detr: value N(0,1); loc U[0,1); attn softmax over the 16 level x point logits.
    tsa:  value N(0,1); loc = reference grid ((j+.5)/200, (i+.5)/200) for q = i*200+j,
          + N(0, 0.01^2); attn softmax over the 4 points.
    sca:  value N(0,1); loc = U[0,1) for 70% and U[-0.2,1.2) for 30% of coordinates
          (draw order: selector, wide, narrow); attn softmax over 32 level x point logits.
    """
    seed, b, shapes, nq, nh, d, npnt = MSDA_CONFIGS[name]
    b = b if batch is None else batch
    nq_full = nq
    nq = max(1, int(round(nq * scale_q)))
    g = torch.Generator().manual_seed(seed)
    spatial_shapes, lsi, s = msda_meta(shapes)
    nl = len(shapes)
    value = torch.randn(b, s, nh, d, generator=g)
    if name == "msda_tsa":
        H, W = shapes[0]
        q = torch.arange(nq_full)[:nq]
        ref = torch.stack([((q % W).double() + 0.5) / W, ((q // W).double() + 0.5) / H], -1)
        loc = ref.float().view(1, nq, 1, 1, 1, 2).expand(b, nq, nh, nl, npnt, 2).clone()
        loc += 0.01 * torch.randn(b, nq, nh, nl, npnt, 2, generator=g)
        attn = torch.softmax(torch.randn(b, nq, nh, nl * npnt, generator=g), -1)
    elif name == "msda_sca":
        shape = (b, nq, nh, nl, npnt, 2)
        sel = torch.rand(shape, generator=g)
        wide = -0.2 + 1.4 * torch.rand(shape, generator=g)
        narrow = torch.rand(shape, generator=g)
        loc = torch.where(sel < 0.3, wide, narrow)
        attn = torch.softmax(torch.randn(b, nq, nh, nl * npnt, generator=g), -1)
    else:
        loc = torch.rand(b, nq, nh, nl, npnt, 2, generator=g)
        attn = torch.softmax(torch.randn(b, nq, nh, nl * npnt, generator=g), -1)
    attn = attn.view(b, nq, nh, nl, npnt)
    return dict(value=value, spatial_shapes=spatial_shapes, level_start_index=lsi,
                sampling_loc=loc.contiguous(), attn_weight=attn.contiguous())


def msda_random(batch, shapes, num_query, heads, head_dim, points, seed=0, loc_lo=-0.1,
                loc_hi=1.1):
    """Small random MSDA problem of any geometry (tests of the generic paths)."""
    g = torch.Generator().manual_seed(seed)
    spatial_shapes, lsi, s = msda_meta(shapes)
    nl = len(shapes)
    value = torch.randn(batch, s, heads, head_dim, generator=g)
    loc = loc_lo + (loc_hi - loc_lo) * torch.rand(batch, num_query, heads, nl, points, 2,
                                                  generator=g)
    attn = torch.softmax(torch.randn(batch, num_query, heads, nl * points, generator=g), -1)
    return dict(value=value, spatial_shapes=spatial_shapes, level_start_index=lsi,
                sampling_loc=loc, attn_weight=attn.view(batch, num_query, heads, nl, points))
