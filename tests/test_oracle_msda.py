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
