"""Pins the MSDA oracle (oracle/msda.py). The reference has no PyTorch golden and no test
vectors for MSDA, so the direct-loop restatement is checked against
  * a scalar brute force of the kernel semantics (tiny pyramids),
  * the F.grid_sample(align_corners=False, padding_mode='zeros') closed form,
  * exact special cases: a pixel-centre location returns that pixel, loc 0 / loc 1 give
    quarter-weight corners, locations past the -1 / H gates give zero,
  * invariants: linearity in value and in attention weights; a constant value map with
    interior locations and weights summing to 1 returns the constant,
  * the committed fixture.
Swapped x/y, a missing -0.5, a dropped corner or a wrong level base fails one of these.
"""
import os

import pytest
import torch

from oracle import inputs
from oracle import msda as om

D64 = torch.float64


def _d64(d):
    return {k: (v.double() if v.is_floating_point() else v) for k, v in d.items()}


@pytest.mark.parametrize("geom", [
    (2, [(5, 6), (3, 4)], 7, 2, 4, 3),
    (1, [(4, 7)], 5, 3, 2, 4),
    (2, [(1, 1), (2, 3), (6, 2)], 4, 1, 3, 2),
])
def test_forward_vs_brute_force(geom):
    d = _d64(inputs.msda_random(*geom, seed=2, loc_lo=-0.4, loc_hi=1.4))
    torch.testing.assert_close(om.forward(**d), om.brute_force(**d), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("cfg", ["msda_detr", "msda_tsa", "msda_sca"])
def test_forward_vs_grid_sample(cfg):
    d = _d64(inputs.msda_inputs(cfg, scale_q=0.003, batch=1))
    torch.testing.assert_close(om.forward(**d), om.forward_grid_sample(**d), rtol=1e-10,
                               atol=1e-12)


def _single(shapes, loc_xy, value, level=0):
    """One query, one head, one point on `level`, attn 1 on it."""
    ss, lsi, s = inputs.msda_meta(shapes)
    L = len(shapes)
    loc = torch.zeros(1, 1, 1, L, 1, 2, dtype=D64)
    loc[0, 0, 0, level, 0] = torch.tensor(loc_xy, dtype=D64)
    attn = torch.zeros(1, 1, 1, L, 1, dtype=D64)
    attn[0, 0, 0, level, 0] = 1.0
    return om.forward(value, ss, lsi, loc, attn)[0, 0]


def test_pixel_centre_returns_pixel():
    shapes = [(3, 5), (4, 7)]
    g = torch.Generator().manual_seed(0)
    value = torch.randn(1, 15 + 28, 1, 6, generator=g, dtype=D64)
    for level, (H, W), start in ((0, (3, 5), 0), (1, (4, 7), 15)):
        for y, x in ((0, 0), (2, 4), (1, 3)):
            if y >= H or x >= W:
                continue
            out = _single(shapes, ((x + 0.5) / W, (y + 0.5) / H), value, level)
            torch.testing.assert_close(out, value[0, start + y * W + x, 0], rtol=1e-14,
                                       atol=1e-14)


def test_corners_at_zero_and_one():
    H, W = 3, 4
    value = torch.randn(1, H * W, 1, 5, dtype=D64)
    torch.testing.assert_close(_single([(H, W)], (0.0, 0.0), value), 0.25 * value[0, 0, 0])
    torch.testing.assert_close(_single([(H, W)], (1.0, 1.0), value), 0.25 * value[0, -1, 0])
    # x = 1 with h_im exactly on row 1: half of that row's last pixel
    out = _single([(H, W)], (1.0, 1.5 / H), value)
    torch.testing.assert_close(out, 0.5 * value[0, 1 * W + W - 1, 0])


@pytest.mark.parametrize("xy", [(-0.5 / 4, 0.5), (0.5, -0.5 / 3), (1 + 0.5 / 4, 0.5),
                                (0.5, 1 + 0.5 / 3), (3.0, 3.0), (-2.0, 0.5)])
def test_gates_give_zero(xy):
    value = torch.randn(1, 12, 1, 3, dtype=D64)
    assert torch.all(_single([(3, 4)], xy, value) == 0)


def test_constant_map_and_linearity():
    d = _d64(inputs.msda_random(2, [(6, 8), (3, 4)], 9, 2, 4, 3, seed=4, loc_lo=0.2,
                                loc_hi=0.8))
    d["attn_weight"] = d["attn_weight"] / d["attn_weight"].sum((-2, -1), keepdim=True)
    const = dict(d, value=torch.full_like(d["value"], 1.75))
    torch.testing.assert_close(om.forward(**const),
                               torch.full((2, 9, 8), 1.75, dtype=D64), rtol=1e-12, atol=1e-12)
    base = om.forward(**d)
    torch.testing.assert_close(om.forward(**dict(d, value=-2 * d["value"])), -2 * base)
    torch.testing.assert_close(om.forward(**dict(d, attn_weight=3 * d["attn_weight"])), 3 * base)


def test_level_start_index_is_used():
    """Moving level 1 by re-packing value changes nothing when lsi moves with it."""
    d = _d64(inputs.msda_random(1, [(3, 4), (2, 3)], 5, 2, 4, 2, seed=6))
    v = d["value"]
    pad = torch.randn(1, 3, 2, 4, dtype=D64)
    v2 = torch.cat([v[:, :12], pad, v[:, 12:]], 1)
    lsi2 = torch.tensor([0, 15])
    torch.testing.assert_close(om.forward(**dict(d, value=v2, level_start_index=lsi2)),
                               om.forward(**d))


def test_fixture():
    fx = torch.load(os.path.join(os.path.dirname(__file__), "golden", "msda_small.pt"),
                    weights_only=True)
    out = om.forward(fx["value"], fx["spatial_shapes"], fx["level_start_index"],
                     fx["sampling_loc"], fx["attn_weight"])
    torch.testing.assert_close(out, fx["out"], rtol=0, atol=0)


# ---------------------------------------------------------------------------------------
# backward: the explicit per-sample restatement against autograd of both forward
# restatements (the direct loop and torch's grid_sample backward) and finite differences.
# A swapped W/H factor, a sign error in one corner term or a missing attention factor
# fails the autograd comparisons.

def _autograd(fwd, d, grad_output):
    v = d["value"].clone().requires_grad_(True)
    loc = d["sampling_loc"].clone().requires_grad_(True)
    a = d["attn_weight"].clone().requires_grad_(True)
    out = fwd(v, d["spatial_shapes"], d["level_start_index"], loc, a)
    gv, gl, ga = torch.autograd.grad(out, (v, loc, a), grad_output, allow_unused=True)
    return gv, gl, ga


@pytest.mark.parametrize("geom", [
    (2, [(5, 6), (3, 4)], 7, 2, 4, 3),
    (1, [(4, 7)], 5, 3, 2, 4),
    (2, [(1, 1), (2, 3), (6, 2)], 4, 1, 3, 2),
])
@pytest.mark.parametrize("fwd", ["loop", "grid_sample"])
def test_backward_vs_autograd(geom, fwd):
    d = _d64(inputs.msda_random(*geom, seed=5, loc_lo=-0.4, loc_hi=1.4))
    B, Lq, NH, L, P, _ = d["sampling_loc"].shape
    D = d["value"].shape[-1]
    g = torch.Generator().manual_seed(9)
    go = torch.randn(B, Lq, NH * D, generator=g, dtype=D64)
    ref = _autograd(om.forward if fwd == "loop" else om.forward_grid_sample, d, go)
    got = om.backward(**d, grad_output=go)
    for r, x in zip(ref, got):
        torch.testing.assert_close(x, r, rtol=1e-11, atol=1e-12)


def test_backward_gradcheck():
    """Finite differences on a tiny pyramid, locations kept off the integer grid lines
    (where the bilinear form has kinks)."""
    d = _d64(inputs.msda_random(1, [(3, 4), (2, 2)], 3, 2, 3, 2, seed=7, loc_lo=-0.3,
                                loc_hi=1.3))
    ss, lsi = d["spatial_shapes"], d["level_start_index"]
    torch.autograd.gradcheck(
        lambda v, loc, a: om.forward(v, ss, lsi, loc, a),
        (d["value"].requires_grad_(True), d["sampling_loc"].requires_grad_(True),
         d["attn_weight"].requires_grad_(True)), eps=1e-6, atol=1e-6)


def test_backward_outside_gate_is_zero():
    """Samples past the -1 / H gates: every gradient is zero."""
    ss, lsi, s = inputs.msda_meta([(4, 5)])
    value = torch.randn(1, s, 1, 3, dtype=D64)
    loc = torch.tensor([[-0.2, 0.5], [0.5, -0.2], [1.2, 0.5], [0.5, 1.3]], dtype=D64)
    loc = loc.view(1, 4, 1, 1, 1, 2)
    attn = torch.ones(1, 4, 1, 1, 1, dtype=D64)
    go = torch.randn(1, 4, 3, dtype=D64)
    gv, gl, ga = om.backward(value, ss, lsi, loc, attn, go)
    assert gv.abs().max() == 0 and gl.abs().max() == 0 and ga.abs().max() == 0


def test_backward_pixel_centre():
    """At a pixel centre all weight is on one corner: grad_value is top*a there, grad_attn
    is top . v(pixel), and grad_loc is W (H) times the one-sided difference toward the
    next column (row)."""
    ss, lsi, s = inputs.msda_meta([(3, 5)])
    g = torch.Generator().manual_seed(1)
    value = torch.randn(1, s, 1, 4, generator=g, dtype=D64)
    y, x = 1, 2
    loc = torch.tensor([(x + 0.5) / 5, (y + 0.5) / 3], dtype=D64).view(1, 1, 1, 1, 1, 2)
    attn = torch.full((1, 1, 1, 1, 1), 0.7, dtype=D64)
    go = torch.randn(1, 1, 4, generator=g, dtype=D64)
    gv, gl, ga = om.backward(value, ss, lsi, loc, attn, go)
    vmap = value[0, :, 0].view(3, 5, 4)
    expect_gv = torch.zeros(3, 5, 4, dtype=D64)
    expect_gv[y, x] = 0.7 * go[0, 0]
    torch.testing.assert_close(gv[0, :, 0].view(3, 5, 4), expect_gv, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(ga.flatten()[0], (go[0, 0] * vmap[y, x]).sum(), rtol=1e-12,
                               atol=1e-12)
    gx = 5 * 0.7 * (go[0, 0] * (vmap[y, x + 1] - vmap[y, x])).sum()
    gy = 3 * 0.7 * (go[0, 0] * (vmap[y + 1, x] - vmap[y, x])).sum()
    torch.testing.assert_close(gl.flatten(), torch.stack([gx, gy]), rtol=1e-12, atol=1e-12)


def test_fp32_coordinates():
    """coord_dtype=float32 is the identity where loc*H - 0.5 is exact in fp32 (loc a
    multiple of 2^-10, H <= 256), and otherwise moves h_im by at most half an fp32 ulp."""
    ss, lsi, s = inputs.msda_meta([(37, 200), (19, 100)])
    g = torch.Generator().manual_seed(4)
    value = torch.randn(1, s, 2, 5, generator=g, dtype=D64)
    loc = (torch.randint(-100, 1124, (1, 6, 2, 2, 3, 2), generator=g) / 1024.0).to(D64)
    attn = torch.rand(1, 6, 2, 2, 3, generator=g, dtype=D64)
    go = torch.randn(1, 6, 10, generator=g, dtype=D64)
    for a, b in zip(om.backward(value, ss, lsi, loc, attn, go, coord_dtype=torch.float32),
                    om.backward(value, ss, lsi, loc, attn, go)):
        torch.testing.assert_close(a, b, rtol=0, atol=0)
    torch.testing.assert_close(om.forward(value, ss, lsi, loc, attn, coord_dtype=torch.float32),
                               om.forward(value, ss, lsi, loc, attn), rtol=0, atol=0)
    loc_h = torch.rand(1000, generator=g, dtype=D64) * 1.4 - 0.2
    h, _ = om._coords(loc_h, loc_h, 200, 200, torch.float32)
    exact = loc_h * 200 - 0.5
    assert ((h - exact).abs() <= torch.abs(exact) * 2.0 ** -24 + 1e-300).all()
    assert (h != exact).any()
