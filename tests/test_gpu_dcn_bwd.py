"""DCNv2 backward on the GPU vs autograd of the float64 oracle (oracle autograd pinned by
gradcheck in test_oracle_dcn.py).

The reference's NHWC per-element backward checks the four corners one by one, its NCHW
backward also applies the -1 / H gate; the two differ only for a sample exactly on h = -1
or w = -1 (which fp16 offsets do hit). The NHWC tests compare with the ungated oracle
(gate=False), the NCHW tests with the gated one. Tolerances as for the forward
(tests/_tol.py), except where stated."""
import pytest
import torch
import torch.nn.functional as F

from _tol import check
from oracle import dcn as od

pytestmark = pytest.mark.gpu
DEV = "cuda"
D64 = torch.float64


def _ext():
    import _modulated_deform_conv_ext
    return _modulated_deform_conv_ext


def _problem(b, cin, h, w, k, s, p, dl, dg=1, cout=8, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    ho, wo = od.out_size(h, p, dl, k, s), od.out_size(w, p, dl, k, s)
    x = torch.randn(b, cin, h, w, generator=g)
    off = 2.0 * torch.randn(b, dg * 2 * k * k, ho, wo, generator=g)
    off.view(-1)[::13] = 40.0
    mask = torch.rand(b, dg * k * k, ho, wo, generator=g)
    weight = 0.1 * torch.randn(cout, cin, k, k, generator=g)
    bias = torch.randn(cout, generator=g)
    r = lambda t: t.to(dtype)
    return r(x), r(off), r(mask), r(weight), r(bias), ho, wo


def _nhwc(t):
    return t.permute(0, 2, 3, 1).contiguous()


# ---------------------------------------------------------------------------------------
# NHWC column-to-image (ext.modulated_deformable_col2im_nhwc_cuda and its variants)
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16],
                         ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("form", ["2T", "3T"])
@pytest.mark.parametrize("geom", [
    # b, cin, h, w, k, stride, pad, dil
    (2, 32, 9, 11, 3, 1, 1, 1),
    (1, 16, 12, 10, 3, 2, 1, 1),
    (1, 64, 8, 9, 3, 1, 2, 2),
    (1, 12, 6, 7, 1, 1, 0, 1),
    # C a multiple of 64: the binned grad_x kernel, with 1, 2 and 4 channels per lane,
    # several output tiles per image, stride 2 and a 5x5 kernel (smaller tiles)
    (1, 128, 21, 30, 3, 1, 1, 1),
    (2, 256, 17, 19, 3, 1, 1, 1),
    (1, 64, 20, 23, 3, 2, 1, 1),
    (1, 64, 13, 14, 5, 1, 2, 1),
])
def test_col2im_nhwc(dtype, form, geom):
    b, cin, h, w, k, s, p, dl = geom
    x, off, mask, _, _, ho, wo = _problem(b, cin, h, w, k, s, p, dl, seed=sum(geom),
                                          dtype=dtype)
    T = k * k
    xh = _nhwc(x)
    g = torch.Generator().manual_seed(1)
    if form == "3T":
        ymask = torch.randn(b, ho, wo, T, generator=g).to(dtype)
        y = torch.cat([_nhwc(off), ymask], dim=-1).contiguous()
        off_arg, mask_arg = y, y
    else:
        off_arg, mask_arg = _nhwc(off), _nhwc(mask)
    M = b * ho * wo
    dcol = torch.randn(M, T * cin, generator=g).to(dtype)
    gx = torch.zeros(b, h, w, cin, device=DEV)
    goff = torch.empty(b, ho, wo, 2 * T, device=DEV)
    gmask = torch.empty(b, ho, wo, T, device=DEV)
    _ext().modulated_deformable_col2im_nhwc_cuda(
        dcol.to(DEV), xh.to(DEV), off_arg.to(DEV), mask_arg.to(DEV), b, cin, h, w, ho, wo, k, k,
        p, p, s, s, dl, dl, 1, gx, goff, gmask)
    torch.cuda.synchronize()
    # oracle: autograd of the columns, weighted by dcol
    xr = xh.double().requires_grad_()
    if form == "3T":
        yr = y.double().requires_grad_()
        o, m = od.split_y_nhwc(yr, T)
        leaves = (xr, yr)
    else:
        o = off_arg.double().requires_grad_()
        m = mask_arg.double().requires_grad_()
        leaves = (xr, o, m)
    cols = od.columns_nhwc(xr, o, m, k, k, s, s, p, p, dl, dl, gate=False)
    grads = torch.autograd.grad((cols * dcol.double()).sum(), leaves)
    check(gx.cpu(), grads[0], torch.float32 if dtype == torch.float32 else dtype, "grad_x")
    if form == "3T":
        check(goff.cpu(), grads[1][..., :2 * T], dtype, "grad_offset")
        check(gmask.cpu(), grads[1][..., 2 * T:], dtype, "grad_mask (pre-sigmoid)")
    else:
        check(goff.cpu(), grads[1], dtype, "grad_offset")
        check(gmask.cpu(), grads[2], dtype, "grad_mask")


def test_col2im_nhwc_partial_outputs():
    """coord-only and grad_x-only variants give the same numbers as the full kernel."""
    x, off, mask, _, _, ho, wo = _problem(1, 32, 10, 10, 3, 1, 1, 1, seed=3)
    b, cin, h, w = x.shape
    ext = _ext()
    args = (1, cin, h, w, ho, wo, 3, 3, 1, 1, 1, 1, 1, 1, 1)
    dcol = torch.randn(ho * wo, 9 * cin).to(DEV)
    xh, oh, mh = (_nhwc(t).to(DEV) for t in (x, off, mask))
    full = [torch.zeros(1, h, w, cin, device=DEV), torch.empty(1, ho, wo, 18, device=DEV),
            torch.empty(1, ho, wo, 9, device=DEV)]
    ext.modulated_deformable_col2im_perelem_nhwc_cuda(dcol, xh, oh, mh, *args, *full)
    co = [torch.empty(1, ho, wo, 18, device=DEV), torch.empty(1, ho, wo, 9, device=DEV)]
    ext.modulated_deformable_col2im_coord_nhwc_cuda(dcol, xh, oh, mh, *args, *co)
    gx = torch.zeros(1, h, w, cin, device=DEV)
    ext.modulated_deformable_gradx_smem_nhwc_cuda(dcol, oh, mh, *args, gx)
    torch.cuda.synchronize()
    assert torch.equal(co[0], full[1]) and torch.equal(co[1], full[2])
    torch.testing.assert_close(gx, full[0], rtol=1e-6, atol=1e-6)  # atomic order differs


# ---------------------------------------------------------------------------------------
# NCHW column-to-image (ext.modulated_deformable_col2im[_coord][_opt|_smem]_cuda)
# ---------------------------------------------------------------------------------------

def _corner_counts(off, b, cin, h, w, k, s, p, dl, dg, ho, wo):
    """Number of (sample, corner) contributions each NCHW input element receives: the
    sampling points of every (pixel, tap) of its deformable group, with the -1 / H gate
    and the per-corner image check of the NCHW kernels. [b, cin, h, w] float64."""
    T = k * k
    o = off.double().view(b, dg, T, 2, ho, wo)
    i = torch.arange(k).repeat_interleave(k).double()
    j = torch.arange(k).repeat(k).double()
    hh = ((torch.arange(ho) * s - p).double().view(1, 1, 1, ho, 1)
          + (i * dl).view(1, 1, T, 1, 1) + o[:, :, :, 0])
    ww = ((torch.arange(wo) * s - p).double().view(1, 1, 1, 1, wo)
          + (j * dl).view(1, 1, T, 1, 1) + o[:, :, :, 1])
    gate = (hh > -1) & (ww > -1) & (hh < h) & (ww < w)
    hl, wl = hh.floor(), ww.floor()
    plane = (torch.arange(b).view(b, 1, 1, 1, 1) * dg + torch.arange(dg).view(1, dg, 1, 1, 1))
    cnt = torch.zeros(b * dg * h * w, dtype=torch.float64)
    for dy in (0, 1):
        for dx in (0, 1):
            y, x = hl + dy, wl + dx
            ok = gate & (y >= 0) & (y < h) & (x >= 0) & (x < w)
            idx = (plane * h * w + y.clamp(0, h - 1).long() * w + x.clamp(0, w - 1).long())
            cnt.index_add_(0, idx.expand_as(ok)[ok], torch.ones(int(ok.sum()), dtype=torch.float64))
    return cnt.view(b, dg, 1, h, w).expand(b, dg, cin // dg, h, w).reshape(b, cin, h, w)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16,
                                   torch.bfloat16], ids=["fp32", "fp64", "fp16", "bf16"])
@pytest.mark.parametrize("geom", [
    # b, cin, h, w, k, stride, pad, dil, dg
    (2, 8, 9, 11, 3, 1, 1, 1, 1),
    (1, 12, 13, 10, 3, 2, 1, 1, 2),
    (2, 6, 12, 12, 3, 1, 2, 2, 3),
    (1, 4, 7, 5, 1, 1, 0, 1, 1),
])
def test_col2im_nchw(dtype, geom):
    b, cin, h, w, k, s, p, dl, dg = geom
    x, off, mask, _, _, ho, wo = _problem(b, cin, h, w, k, s, p, dl, dg=dg, seed=sum(geom),
                                          dtype=dtype)
    T = k * k
    g = torch.Generator().manual_seed(2)
    col = torch.randn(cin * T, b * ho * wo, generator=g).to(dtype)
    ext = _ext()
    args = (b, cin, h, w, ho, wo, k, k, p, p, s, s, dl, dl, dg)
    gx = torch.zeros(b, cin, h, w, dtype=dtype, device=DEV)
    ext.modulated_deformable_col2im_smem_cuda(col.to(DEV), off.to(DEV), mask.to(DEV), *args, gx)
    goff = torch.empty(off.shape, dtype=dtype, device=DEV)
    gmask = torch.empty(mask.shape, dtype=dtype, device=DEV)
    ext.modulated_deformable_col2im_coord_opt_cuda(col.to(DEV), x.to(DEV), off.to(DEV),
                                                   mask.to(DEV), *args, goff, gmask)
    torch.cuda.synchronize()
    xr, o, m = (t.double().requires_grad_() for t in (x, off, mask))
    cols = od.im2col_nchw(xr, o, m, k, k, p, p, s, s, dl, dl, dg)
    gr = torch.autograd.grad((cols * col.double().view(cols.shape)).sum(), (xr, o, m))
    # grad_x is accumulated by atomics in the input dtype (the reference's col2im kernels
    # do the same), in an order that changes from run to run. For bf16 every one of an
    # element's n adds rounds the running sum (unit roundoff u = 2^-8), and so may the
    # term itself: |error| <= (n + 1) u sum|terms|, where sum|terms| is the same gradient
    # taken with |col| (bilinear weights and masks are >= 0) and n counts the element's
    # (sample, corner) contributions.
    if dtype == torch.bfloat16:
        r = gr[0]
        xa = x.double().requires_grad_()
        ca = od.im2col_nchw(xa, off.double(), mask.double(), k, k, p, p, s, s, dl, dl, dg)
        r_abs = torch.autograd.grad((ca * col.double().abs().view(ca.shape)).sum(), xa)[0]
        n = _corner_counts(off, b, cin, h, w, k, s, p, dl, dg, ho, wo)
        err = (gx.cpu().double() - r).abs()
        bound = (n + 1) * 2.0 ** -8 * r_abs * 1.01 + 1e-6
        assert (err <= bound).all(), f"bf16 grad_x: max err / bound {(err / bound).max():.3f}"
    else:
        check(gx.cpu(), gr[0], dtype, "grad_x")
    check(goff.cpu(), gr[1], dtype, "grad_offset")
    check(gmask.cpu(), gr[2], dtype, "grad_mask")


# ---------------------------------------------------------------------------------------
# Autograd functions
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("groups,dg", [(1, 1), (2, 1), (1, 2)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16],
                         ids=["fp32", "fp64", "fp16"])
def test_modulated_deform_conv2d_backward(groups, dg, dtype):
    from modulated_deform_conv import modulated_deform_conv2d
    g = torch.Generator().manual_seed(groups * 10 + dg)
    b, cin, cout, h, w = 2, 16, 24, 9, 10
    x = torch.randn(b, cin, h, w, generator=g)
    off = 2.0 * torch.randn(b, dg * 18, h, w, generator=g)
    mask = torch.rand(b, dg * 9, h, w, generator=g)
    weight = 0.1 * torch.randn(cout, cin // groups, 3, 3, generator=g)
    bias = torch.randn(cout, generator=g)
    go = torch.randn(b, cout, h, w, generator=g)
    leaves = [t.to(dtype).to(DEV).requires_grad_() for t in (x, off, mask, weight, bias)]
    out = modulated_deform_conv2d(*leaves, 1, 1, 1, groups, dg)
    out.backward(go.to(dtype).to(DEV))
    torch.cuda.synchronize()
    ref_leaves = [t.to(dtype).double().requires_grad_() for t in (x, off, mask, weight, bias)]
    ref = od.forward_nchw(*ref_leaves, (1, 1), (1, 1), (1, 1), groups, dg)
    ref.backward(go.to(dtype).double())
    tol = torch.float32 if dtype != torch.float16 else dtype
    for name, a, r in zip(("x", "offset", "mask", "weight", "bias"), leaves, ref_leaves):
        check(a.grad.cpu(), r.grad, tol, f"grad {name} g{groups} dg{dg}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
@pytest.mark.parametrize("bn,relu", [(False, False), (True, False), (True, True)])
def test_dcn_split_nhwc_backward(dtype, bn, relu):
    from modulated_deform_conv import dcn_split_nhwc as dsn
    g = torch.Generator().manual_seed(5)
    b, h, w, cin, cout = 2, 10, 12, 32, 48
    x = torch.randn(b, h, w, cin, generator=g)
    w_off = 0.05 * torch.randn(27, cin, 3, 3, generator=g)
    b_off = 0.3 * torch.randn(27, generator=g)
    weight = 0.1 * torch.randn(cout, cin, 3, 3, generator=g)
    bias = torch.randn(cout, generator=g)
    scale = 0.5 + torch.rand(cout, generator=g) if bn else None
    shift = torch.randn(cout, generator=g) if bn else None
    go = torch.randn(b, h, w, cout, generator=g)
    leaves = [t.to(dtype).to(DEV).requires_grad_() for t in (x, w_off, b_off, weight, bias)]
    out = dsn.dcn_split_nhwc(*leaves, 1, 1, 1,
                             None if scale is None else scale.to(DEV),
                             None if shift is None else shift.to(DEV), relu)
    out.backward(go.to(dtype).to(DEV))
    torch.cuda.synchronize()
    # float64 reference of the same composition, by autograd. The derivative of a bilinear
    # sample with respect to its position jumps at cell edges, so the reference evaluates
    # it at the kernel's own sample positions: the forward value of y is the one the
    # backward reads (the kernel's fp32 offset conv rounded to the input dtype), its
    # gradient that of the exact conv.
    r = [t.to(dtype).double().requires_grad_() for t in (x, w_off, b_off, weight, bias)]
    y = F.conv2d(r[0].permute(0, 3, 1, 2), r[1], r[2], 1, 1, 1)
    with torch.no_grad():
        assert dsn.mega_supported(leaves[0], leaves[1], leaves[3])
        y_kernel = dsn.offset_conv_y(leaves[0], leaves[1], leaves[2], 1, 1, 1).to(dtype)
    y = y + (y_kernel.permute(0, 3, 1, 2).cpu().double() - y).detach()
    y = y.permute(0, 2, 3, 1)
    o, m = od.split_y_nhwc(y, 9)
    ref = od.forward_nhwc(r[0], o, m, r[3], r[4], 1, 1, 1, gate=False)
    if bn:
        ref = ref * scale.double() + shift.double()
        if relu:
            # the backward takes the ReLU mask the forward saved (dcn_split_nhwc.py:
            # 190-196, 245-250): outputs within rounding of 0 follow the kernel's sign
            ref = ref * (out.detach().cpu() > 0)
    ref.backward(go.to(dtype).double())
    tol_dtype = torch.float32 if dtype == torch.float32 else dtype
    for name, a, rr in zip(("x", "w_off", "b_off", "weight", "bias"), leaves, r):
        check(a.grad.cpu(), rr.grad, tol_dtype, f"grad {name} bn{bn} relu{relu}")


# ---------------------------------------------------------------------------------------
# fused_tl backward: dcn_col2im_nhwc and the autograd dcn_split / Pack(backend='tilelang')
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_fused_tl_col2im_nhwc(dtype):
    """fused_tl.dcn_col2im_nhwc (fused_tl.py:831-862): fp32 gradients of X, offset and the
    (post-sigmoid) mask, against autograd of the oracle columns weighted by dCol."""
    from modulated_deform_conv import fused_tl
    x, off, mask, _, _, ho, wo = _problem(2, 64, 11, 13, 3, 1, 1, 1, seed=8, dtype=dtype)
    b, cin, h, w = x.shape
    xh, oh, mh = _nhwc(x), _nhwc(off), _nhwc(mask)
    g = torch.Generator().manual_seed(2)
    dcol = torch.randn(b * ho * wo, 9 * cin, generator=g).to(dtype)
    gx, goff, gmask = fused_tl.dcn_col2im_nhwc(dcol.to(DEV), xh.to(DEV), oh.to(DEV),
                                               mh.to(DEV), 3, 3, 1, 1, 1)
    torch.cuda.synchronize()
    assert gx.dtype == goff.dtype == gmask.dtype == torch.float32
    leaves = [t.double().requires_grad_() for t in (xh, oh, mh)]
    cols = od.columns_nhwc(*leaves, 3, 3, 1, 1, 1, 1, 1, 1, gate=False)
    grads = torch.autograd.grad((cols * dcol.double()).sum(), leaves)
    tol = torch.float32 if dtype == torch.float32 else dtype
    for name, a, r in zip(("grad_X", "grad_offset", "grad_mask"), (gx, goff, gmask), grads):
        check(a.cpu(), r, tol, f"dcn_col2im_nhwc {name}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_pack_tilelang_backward(dtype):
    """ModulatedDeformConv2dPack(backend='tilelang') trains: fused_tl.dcn_apply_nchw ->
    _DCNSplitFunction. Gradients of the input and of all four parameters against autograd
    of the float64 oracle evaluated at the kernel's sample positions (see
    test_dcn_split_nhwc_backward)."""
    from modulated_deform_conv import ModulatedDeformConv2dPack
    from modulated_deform_conv import dcn_split_nhwc as dsn
    torch.manual_seed(3)
    mod = ModulatedDeformConv2dPack(64, 48, 3, stride=1, padding=1, backend="tilelang")
    with torch.no_grad():
        mod.conv_offset.weight.normal_(0, 0.03)
        mod.conv_offset.bias.normal_(0, 0.5)
        mod.bias.normal_()
    mod = mod.to(dtype).to(DEV)
    x = torch.randn(2, 64, 9, 10).to(dtype).to(DEV).requires_grad_()
    out = mod(x)
    g = torch.Generator().manual_seed(4)
    go = torch.randn(out.shape, generator=g).to(dtype)
    out.backward(go.to(DEV))
    torch.cuda.synchronize()
    params = [mod.conv_offset.weight, mod.conv_offset.bias, mod.weight, mod.bias]
    r = [t.detach().cpu().double().requires_grad_() for t in [x] + params]
    xr = r[0].permute(0, 2, 3, 1)
    y = F.conv2d(r[0], r[1], r[2], 1, 1, 1)
    with torch.no_grad():
        xk = x.detach().permute(0, 2, 3, 1).contiguous()
        y_kernel = dsn.offset_conv_y(xk, mod.conv_offset.weight, mod.conv_offset.bias, 1, 1,
                                     1).to(dtype)
    y = (y + (y_kernel.permute(0, 3, 1, 2).cpu().double() - y).detach()).permute(0, 2, 3, 1)
    o, m = od.split_y_nhwc(y, 9)
    ref = od.forward_nhwc(xr, o, m, r[3], r[4], 1, 1, 1, gate=False).permute(0, 3, 1, 2)
    ref.backward(go.double())
    tol = torch.float32 if dtype == torch.float32 else dtype
    for name, a, rr in zip(("x", "w_off", "b_off", "weight", "bias"), [x] + params, r):
        check(a.grad.cpu(), rr.grad, tol, f"tilelang Pack grad {name}")
