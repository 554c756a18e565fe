"""Pins the DCNv2 oracle (oracle/dcn.py) without the reference's code: the reference
ships no golden vectors or tests for this path, so each oracle function is checked
against
  * a scalar brute force of the DCNv2 definition (tiny shapes, special offsets),
  * closed forms through F.conv2d: zero offsets with unit mask are a plain convolution,
    a constant integer offset is a convolution of the shifted zero-padded image,
  * special cases: mask 0 -> bias; half-pixel offsets average two neighbours; the
    -1 / H gates; linearity in x and in mask,
  * the NCHW and NHWC restatements against each other,
  * the committed fixture of BASELINE configs[0].
A dropped corner, swapped (dy, dx), wrong gate or transposed K order fails one of these.
"""
import os

import pytest
import torch
import torch.nn.functional as F

from oracle import dcn as od
from oracle import inputs

D64 = torch.float64


def _problem(b, c, h, w, cout, kh=3, kw=3, dg=1, groups=1, stride=1, pad=1, dil=1, seed=0,
             off_std=1.5):
    g = torch.Generator().manual_seed(seed)
    ho = od.out_size(h, pad, dil, kh, stride)
    wo = od.out_size(w, pad, dil, kw, stride)
    x = torch.randn(b, c, h, w, generator=g, dtype=D64)
    off = off_std * torch.randn(b, dg * 2 * kh * kw, ho, wo, generator=g, dtype=D64)
    off.view(-1)[::5] = torch.round(off.view(-1)[::5])          # integer landings
    off.view(-1)[::9] = torch.round(off.view(-1)[::9]) + 0.5    # half pixels
    off.view(-1)[::17] = -30.0                                   # far outside
    mask = torch.rand(b, dg * kh * kw, ho, wo, generator=g, dtype=D64)
    weight = torch.randn(cout, c // groups, kh, kw, generator=g, dtype=D64)
    bias = torch.randn(cout, generator=g, dtype=D64)
    return x, off, mask, weight, bias, (stride, stride), (pad, pad), (dil, dil)


@pytest.mark.parametrize("geom", [
    dict(b=2, c=4, h=5, w=6, cout=3),
    dict(b=1, c=4, h=6, w=5, cout=4, dg=2),
    dict(b=1, c=4, h=7, w=7, cout=4, groups=2),
    dict(b=1, c=3, h=7, w=6, cout=2, stride=2),
    dict(b=1, c=2, h=8, w=7, cout=2, dil=2, pad=2),
    dict(b=1, c=2, h=5, w=5, cout=3, kh=1, kw=1, pad=0),
    dict(b=1, c=2, h=6, w=5, cout=2, kh=3, kw=2, pad=1),
])
def test_forward_nchw_vs_brute_force(geom):
    kh, kw = geom.get("kh", 3), geom.get("kw", 3)
    x, off, m, w, b, s, p, d = _problem(geom["b"], geom["c"], geom["h"], geom["w"],
                                        geom["cout"], kh, kw, geom.get("dg", 1),
                                        geom.get("groups", 1), geom.get("stride", 1),
                                        geom.get("pad", 1), geom.get("dil", 1), seed=len(geom))
    dg, groups = geom.get("dg", 1), geom.get("groups", 1)
    got = od.forward_nchw(x, off, m, w, b, s, p, d, groups, dg)
    want = od.brute_force_nchw(x, off, m, w, b, s, p, d, dg)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("stride,pad,dil,groups", [(1, 1, 1, 1), (2, 1, 1, 1), (1, 2, 2, 1),
                                                   (1, 1, 1, 2), (2, 0, 1, 4)])
def test_zero_offset_unit_mask_is_conv2d(stride, pad, dil, groups):
    x, off, m, w, b, s, p, d = _problem(2, 8, 11, 9, 8, groups=groups, stride=stride, pad=pad,
                                        dil=dil, seed=3)
    off.zero_()
    m.fill_(1.0)
    got = od.forward_nchw(x, off, m, w, b, s, p, d, groups, 1)
    want = F.conv2d(x, w, b, s, p, d, groups)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dy,dx", [(1, -2), (-3, 0), (2, 5), (0, 1)])
def test_integer_shift_is_conv_of_shifted_image(dy, dx):
    x, off, m, w, b, s, p, d = _problem(1, 3, 9, 10, 4, seed=5)
    off.view(1, 9, 2, *off.shape[-2:])[:, :, 0] = float(dy)
    off.view(1, 9, 2, *off.shape[-2:])[:, :, 1] = float(dx)
    m.fill_(1.0)
    got = od.forward_nchw(x, off, m, w, b, s, p, d)
    # A deformable tap samples the zero-extended image X at oh - p + i + dy, even when
    # oh - p + i itself lies in the padding. So: zero-extend by a margin M, cut the
    # window that starts at (dy - p, dx - p) and run an unpadded convolution on it.
    H, W = x.shape[-2:]
    M, pad = 8, p[0]
    big = F.pad(x, (M, M, M, M))               # big[r, c] = X[r - M, c - M]
    win = big[..., M + dy - pad:M + dy - pad + H + 2 * pad, M + dx - pad:M + dx - pad + W + 2 * pad]
    want = F.conv2d(win, w, b, s, 0, d)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


def test_mask_zero_gives_bias():
    x, off, m, w, b, s, p, d = _problem(2, 4, 6, 7, 5, seed=7)
    got = od.forward_nchw(x, off, torch.zeros_like(m), w, b, s, p, d)
    torch.testing.assert_close(got, b.view(1, -1, 1, 1).expand_as(got), rtol=0, atol=1e-14)


def test_half_pixel_averages_neighbours():
    """1x1 kernel, dy = 0.5: the tap is the mean of rows y and y+1 (the last row sees half
    of itself and a zero neighbour)."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 1, 5, 4, generator=g, dtype=D64)
    off = torch.zeros(1, 2, 5, 4, dtype=D64)
    off[:, 0] = 0.5
    col = od.im2col_nchw(x, off, torch.ones(1, 1, 5, 4, dtype=D64), 1, 1, 0, 0, 1, 1, 1, 1, 1)
    xp = torch.cat([x[0, 0], torch.zeros(1, 4, dtype=D64)], 0)
    torch.testing.assert_close(col[0, 0], 0.5 * (xp[:-1] + xp[1:]), rtol=1e-15, atol=1e-15)


def test_gates_at_minus_one_and_h():
    """h = -1 or h = H contributes 0; h = H-1 (integer) returns the last row exactly."""
    x = torch.arange(1, 13, dtype=D64).view(1, 1, 3, 4)
    ones = torch.ones(1, 1, 3, 4, dtype=D64)
    for dy, want_row in ((-1.0, None), (3.0, None), (-1.0 + 1e-9, 0)):
        off = torch.zeros(1, 2, 3, 4, dtype=D64)
        off[:, 0, 0] = dy                     # output row 0 samples h = dy
        col = od.im2col_nchw(x, off, ones, 1, 1, 0, 0, 1, 1, 1, 1, 1)[0, 0, 0]
        if want_row is None:
            assert torch.all(col == 0)
        else:
            torch.testing.assert_close(col, x[0, 0, 0] * 1e-9, rtol=1e-6, atol=1e-12)
    off = torch.zeros(1, 2, 3, 4, dtype=D64)
    off[:, 0, 0] = 2.0
    col = od.im2col_nchw(x, off, ones, 1, 1, 0, 0, 1, 1, 1, 1, 1)[0, 0, 0]
    torch.testing.assert_close(col, x[0, 0, 2], rtol=0, atol=0)


def test_linearity():
    x, off, m, w, b, s, p, d = _problem(1, 4, 7, 6, 3, seed=9)
    base = od.forward_nchw(x, off, m, w, None, s, p, d)
    torch.testing.assert_close(od.forward_nchw(3 * x, off, m, w, None, s, p, d), 3 * base)
    torch.testing.assert_close(od.forward_nchw(x, off, 0.25 * m, w, None, s, p, d), 0.25 * base)


def test_fused_front_end_reduces_to_constant_offsets():
    """w_off = 0: y is b_off everywhere, so the front end is the NHWC columns with one
    constant (dy, dx) per tap and mask sigmoid(b); a weight on one input channel moves the
    offsets by that channel's conv."""
    g = torch.Generator().manual_seed(14)
    x = torch.randn(2, 7, 6, 5, generator=g, dtype=D64)
    T = 9
    b_off = torch.randn(3 * T, generator=g, dtype=D64)
    w0 = torch.zeros(3 * T, T, 5, dtype=D64)
    cols = od.fused_front_end_columns(x, w0, b_off, 3, 3, 1, 1, 1)
    off = b_off[:2 * T].expand(2, 7, 6, 2 * T)
    msk = torch.sigmoid(b_off[2 * T:]).expand(2, 7, 6, T)
    torch.testing.assert_close(cols, od.columns_nhwc(x, off, msk, 3, 3, 1, 1, 1, 1, 1, 1),
                               rtol=0, atol=0)
    # centre-tap weight 1 on channel 0 for the dy of tap 4: dy = x[..., 0] + b
    w1 = w0.clone()
    w1[8, 4, 0] = 1.0
    cols = od.fused_front_end_columns(x, w1, b_off, 3, 3, 1, 1, 1)
    off2 = off.clone()
    off2[..., 8] = off2[..., 8] + x[..., 0]
    torch.testing.assert_close(cols, od.columns_nhwc(x, off2, msk, 3, 3, 1, 1, 1, 1, 1, 1),
                               rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("col_dtype", [torch.float16, torch.bfloat16])
def test_column_rounding(col_dtype):
    """col_dtype rounds each column once: exact columns are unchanged, and in general the
    output moves by at most one half-ulp of every column times |weight|."""
    g = torch.Generator().manual_seed(12)
    x = torch.randint(-4, 5, (1, 4, 6, 7), generator=g).to(D64)
    off = torch.randint(-2, 3, (1, 18, 6, 7), generator=g).to(D64)     # integer landings
    m = torch.ones(1, 9, 6, 7, dtype=D64)
    w = torch.randn(5, 4, 3, 3, generator=g, dtype=D64)
    args = ((1, 1), (1, 1), (1, 1))
    torch.testing.assert_close(od.forward_nchw(x, off, m, w, None, *args, col_dtype=col_dtype),
                               od.forward_nchw(x, off, m, w, None, *args), rtol=0, atol=0)
    x, off, m, w, b, s, p, d = _problem(1, 4, 7, 6, 3, seed=13)
    exact = od.forward_nchw(x, off, m, w, None, s, p, d)
    rounded = od.forward_nchw(x, off, m, w, None, s, p, d, col_dtype=col_dtype)
    cols = od.im2col_nchw(x, off, m, 3, 3, 1, 1, 1, 1, 1, 1, 1)
    half_ulp = 2.0 ** -(11 if col_dtype == torch.float16 else 8)
    bound = half_ulp * (w.reshape(3, -1).abs() @ cols.abs().reshape(36, -1))
    diff = (rounded - exact).permute(1, 0, 2, 3).reshape(3, -1)
    assert (diff.abs() <= bound.reshape(3, -1) + 1e-12).all()
    assert (diff != 0).any()                                            # rounding happened
    nhwc = od.forward_nhwc(x.permute(0, 2, 3, 1), off.permute(0, 2, 3, 1),
                           m.permute(0, 2, 3, 1), w, None, 1, 1, 1, col_dtype=col_dtype)
    torch.testing.assert_close(nhwc.permute(0, 3, 1, 2), rounded, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("stride,pad,dil", [(1, 1, 1), (2, 1, 1), (1, 2, 2)])
def test_nchw_and_nhwc_restatements_agree(stride, pad, dil):
    x, off, m, w, b, s, p, d = _problem(2, 6, 9, 8, 5, stride=stride, pad=pad, dil=dil, seed=11)
    nchw = od.forward_nchw(x, off, m, w, b, s, p, d)
    nhwc = od.forward_nhwc(x.permute(0, 2, 3, 1), off.permute(0, 2, 3, 1),
                           m.permute(0, 2, 3, 1), w, b, stride, pad, dil)
    torch.testing.assert_close(nhwc.permute(0, 3, 1, 2), nchw, rtol=1e-12, atol=1e-12)
    # columns: NHWC k = t*C + c  <->  NCHW row c*T + t
    cols_nhwc = od.columns_nhwc(x.permute(0, 2, 3, 1), off.permute(0, 2, 3, 1),
                                m.permute(0, 2, 3, 1), 3, 3, stride, stride, pad, pad, dil, dil)
    cols_nchw = od.im2col_nchw(x, off, m, 3, 3, pad, pad, stride, stride, dil, dil, 1)
    C, T = 6, 9
    a = cols_nhwc.view(-1, T, C).permute(2, 1, 0).reshape(C * T, -1)
    torch.testing.assert_close(a, cols_nchw.reshape(C * T, -1), rtol=0, atol=0)


def test_pack_offset_split_conventions():
    """NCHW Pack split (chunk -> cat(o1, o2), sigmoid(o3)) == NHWC y split after permute."""
    y = torch.randn(2, 27, 4, 5, dtype=D64)
    o_nchw, m_nchw = od.split_y_nchw(y, 9)
    o_nhwc, m_nhwc = od.split_y_nhwc(y.permute(0, 2, 3, 1), 9)
    torch.testing.assert_close(o_nhwc, o_nchw.permute(0, 2, 3, 1), rtol=0, atol=0)
    torch.testing.assert_close(m_nhwc, m_nchw.permute(0, 2, 3, 1), rtol=0, atol=0)


def test_config1_fixture():
    fx = torch.load(os.path.join(os.path.dirname(__file__), "golden", "dcn_c1.pt"),
                    weights_only=True)
    d = inputs.dcn_inputs("dcn_c1")
    for k, v in fx["checksums"].items():
        assert abs(float(d[k].double().sum() + (d[k].double() ** 2).sum()) - v) < 1e-6 * abs(v)
    out = od.forward_nchw(d["x"].double(), d["offset"].double(), d["mask"].double(),
                          d["weight"].double(), d["bias"].double(), d["stride"], d["padding"],
                          d["dilation"])
    torch.testing.assert_close(out.float(), fx["out"], rtol=0, atol=0)


def test_package_pytorch_goldens_match_oracle():
    """The package's pure-PyTorch implementations (public API of the reference) agree with
    the oracle; they are not used as the checker anywhere."""
    from modulated_deform_conv import modulated_deform_conv as mdc
    from modulated_deform_conv import fused_tl
    x, off, m, w, b, s, p, d = _problem(2, 4, 7, 8, 3, dg=2, seed=13)
    got = mdc.modulated_deformable_im2col_pytorch(x, off, m, 3, 3, 1, 1, 1, 1, 1, 1, 2)
    torch.testing.assert_close(got, od.im2col_nchw(x, off, m, 3, 3, 1, 1, 1, 1, 1, 1, 2))
    x, off, m, w, b, s, p, d = _problem(2, 4, 7, 8, 3, seed=14)
    xn, on, mn = (t.permute(0, 2, 3, 1) for t in (x, off, m))
    torch.testing.assert_close(fused_tl.dcn_forward_golden_nhwc(xn, on, mn, w, b, 1, 1, 1),
                               od.forward_nhwc(xn, on, mn, w, b, 1, 1, 1))


# ---------------------------------------------------------------------------------------
# Gradients: the backward kernels are checked against autograd of these restatements, so
# autograd of the restatements is pinned here against finite differences (gradcheck).
# Offsets are continuous (no sample on a cell edge, where the derivative jumps).
# ---------------------------------------------------------------------------------------

def _smooth_problem(seed, b=1, c=3, h=5, w=6, cout=2, k=3, dg=1):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, c, h, w, generator=g, dtype=D64)
    off = 1.3 * torch.randn(b, dg * 2 * k * k, h, w, generator=g, dtype=D64)
    mask = torch.rand(b, dg * k * k, h, w, generator=g, dtype=D64)
    weight = torch.randn(cout, c, k, k, generator=g, dtype=D64)
    return x, off, mask, weight


def test_gradcheck_forward_nchw():
    x, off, mask, weight = _smooth_problem(21, dg=1)
    f = lambda x, off, mask, weight: od.forward_nchw(x, off, mask, weight, None, (1, 1), (1, 1),
                                                     (1, 1))
    assert torch.autograd.gradcheck(f, (x.requires_grad_(), off.requires_grad_(),
                                        mask.requires_grad_(), weight.requires_grad_()))


def test_ungated_columns_equal_gated_values():
    """gate=False changes no value (a sample outside (-1, H) x (-1, W) has no in-range
    corner with a non-zero weight); only the derivative exactly at -1 differs."""
    x, off, mask, w, b, s, p, d = _problem(2, 4, 7, 8, 3, seed=24)
    args = (x.permute(0, 2, 3, 1), off.permute(0, 2, 3, 1), mask.permute(0, 2, 3, 1), 3, 3,
            1, 1, 1, 1, 1, 1)
    torch.testing.assert_close(od.columns_nhwc(*args, gate=False), od.columns_nhwc(*args),
                               rtol=0, atol=0)
    # one sample exactly on h = -1: value 0 both ways, derivative 0 (gated) vs one-sided
    xx = torch.randn(1, 3, 3, 2, dtype=D64)
    h = torch.tensor([-1.0], dtype=D64, requires_grad=True)
    w = torch.tensor([0.5], dtype=D64)
    g_on = torch.autograd.grad(od.bilinear_nhwc(xx[0], h, w).sum(), h)[0]
    h2 = h.detach().clone().requires_grad_()
    v = od.bilinear_nhwc(xx[0], h2, w, gate=False)
    g_off = torch.autograd.grad(v.sum(), h2)[0]
    assert g_on.item() == 0.0 and float(v.detach().abs().sum()) == 0.0
    # cell [-1, 0]: d/dh = (1 - lw) * x[0, 0] + lw * x[0, 1] summed over channels
    expect = (0.5 * xx[0, 0, 0] + 0.5 * xx[0, 0, 1]).sum()
    torch.testing.assert_close(g_off[0], expect)


def test_gradcheck_columns_nhwc():
    x, off, mask, _ = _smooth_problem(22)
    f = lambda x, off, mask: od.columns_nhwc(x, off, mask, 3, 3, 1, 1, 1, 1, 1, 1)
    args = (x.permute(0, 2, 3, 1).contiguous().requires_grad_(),
            off.permute(0, 2, 3, 1).contiguous().requires_grad_(),
            mask.permute(0, 2, 3, 1).contiguous().requires_grad_())
    assert torch.autograd.gradcheck(f, args)


def test_gradcheck_front_end_columns():
    g = torch.Generator().manual_seed(23)
    x = torch.randn(1, 4, 5, 3, generator=g, dtype=D64)
    w_off = 0.3 * torch.randn(27, 9, 3, generator=g, dtype=D64)
    b_off = torch.randn(27, generator=g, dtype=D64)
    f = lambda x, w, b: od.fused_front_end_columns(x, w, b, 3, 3, 1, 1, 1)
    assert torch.autograd.gradcheck(f, (x.requires_grad_(), w_off.requires_grad_(),
                                        b_off.requires_grad_()))


def test_fp32_coordinates():
    """coord_dtype=torch.float32 evaluates the sample at fp32(tap position + offset):
    (1) offsets whose sum with the tap position is exact in fp32 leave the columns
    unchanged; (2) an offset that needs more than 24 bits (39 - 0.00172901153...) gives
    the columns of the explicitly rounded coordinate, and so a different value from the
    exact one; (3) gradients flow to the offset as through the identity."""
    g = torch.Generator().manual_seed(6)
    x = torch.randn(1, 6, 45, 3, generator=g, dtype=torch.float64)
    off = torch.round(4 * torch.randn(1, 6, 45, 18, generator=g, dtype=torch.float64)) / 256
    mask = torch.rand(1, 6, 45, 9, generator=g, dtype=torch.float64)
    exact = od.columns_nhwc(x, off, mask, 3, 3, 1, 1, 1, 1, 1, 1)
    rounded = od.columns_nhwc(x, off, mask, 3, 3, 1, 1, 1, 1, 1, 1, coord_dtype=torch.float32)
    assert torch.equal(exact, rounded)
    # pixel (0, 40), tap t = 3 (ki = 1, kj = 0): w = 40 - 1 + 0 + dx = 39 + dx
    dx = -0.0017290115356445312            # an fp16 value; 39 + dx is not an fp32
    off2 = off.clone()
    off2[0, 0, 40, 2 * 3 + 1] = dx
    w32 = float(torch.tensor(39.0 + dx, dtype=torch.float64).float())
    assert w32 != 39.0 + dx
    off3 = off2.clone()
    off3[0, 0, 40, 2 * 3 + 1] = w32 - 39.0  # exact in float64: the rounded coordinate
    got = od.columns_nhwc(x, off2, mask, 3, 3, 1, 1, 1, 1, 1, 1, coord_dtype=torch.float32)
    want = od.columns_nhwc(x, off3, mask, 3, 3, 1, 1, 1, 1, 1, 1)
    assert torch.equal(got, want)
    assert not torch.equal(got, od.columns_nhwc(x, off2, mask, 3, 3, 1, 1, 1, 1, 1, 1))
    o = off2.clone().requires_grad_()
    od.columns_nhwc(x, o, mask, 3, 3, 1, 1, 1, 1, 1, 1, coord_dtype=torch.float32).sum().backward()
    o3 = off3.clone().requires_grad_()
    od.columns_nhwc(x, o3, mask, 3, 3, 1, 1, 1, 1, 1, 1).sum().backward()
    assert torch.allclose(o.grad, o3.grad, rtol=0, atol=1e-12)
