"""DCNv2 forward on the GPU vs the float64 CPU oracle (oracle/dcn.py), through the
reference-shaped APIs: the extension functions (_modulated_deform_conv_ext), the NHWC
entry points (fused_tl / dcn_split_nhwc) and the modules (modulated_deform_conv).

Full-size ResNet-101 res4/res5 configurations run whole on the GPU; the oracle checks
the first and last image."""
import pytest
import torch
import torch.nn.functional as F

from _tol import check
from oracle import dcn as od
from oracle import inputs

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
HALF = [torch.float16, torch.bfloat16]


def _ext():
    import _modulated_deform_conv_ext
    return _modulated_deform_conv_ext


def _rand_problem(b, cin, cout, h, w, k=3, stride=1, pad=1, dil=1, dg=1, groups=1, seed=0,
                  off_std=2.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    ho = od.out_size(h, pad, dil, k, stride)
    wo = od.out_size(w, pad, dil, k, stride)
    x = torch.randn(b, cin, h, w, generator=g)
    off = off_std * torch.randn(b, dg * 2 * k * k, ho, wo, generator=g)
    # a few taps exactly on integers, half pixels and far outside
    off.view(-1)[::7] = torch.round(off.view(-1)[::7])
    off.view(-1)[::11] = torch.round(off.view(-1)[::11]) + 0.5
    off.view(-1)[::13] = 40.0
    mask = torch.rand(b, dg * k * k, ho, wo, generator=g)
    weight = 0.1 * torch.randn(cout, cin // groups, k, k, generator=g)
    bias = torch.randn(cout, generator=g)
    r = lambda t: t.to(dtype)
    return dict(x=r(x), offset=r(off), mask=r(mask), weight=r(weight), bias=r(bias),
                stride=(stride, stride), padding=(pad, pad), dilation=(dil, dil), dg=dg,
                groups=groups)


# ---------------------------------------------------------------------------------------
# NCHW columns (ext.modulated_deformable_im2col[_opt]_cuda)
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("entry", ["modulated_deformable_im2col_cuda",
                                   "modulated_deformable_im2col_opt_cuda"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16, torch.bfloat16],
                         ids=["fp32", "fp64", "fp16", "bf16"])
@pytest.mark.parametrize("geom", [
    # b, cin, h, w, k, stride, pad, dil, dg
    (2, 8, 9, 11, 3, 1, 1, 1, 1),
    (1, 12, 13, 10, 3, 2, 1, 1, 2),
    (2, 6, 12, 12, 3, 1, 2, 2, 3),
    (1, 4, 7, 5, 1, 1, 0, 1, 1),
    (1, 64, 32, 32, 3, 1, 1, 1, 1),
])
def test_im2col_nchw(entry, dtype, geom):
    b, cin, h, w, k, s, p, dl, dg = geom
    d = _rand_problem(b, cin, 4, h, w, k, s, p, dl, dg, dtype=dtype, seed=sum(geom))
    ho, wo = od.out_size(h, p, dl, k, s), od.out_size(w, p, dl, k, s)
    col = torch.full((cin * k * k, b, ho, wo), float("nan"), dtype=dtype, device=DEV)
    getattr(_ext(), entry)(d["x"].to(DEV), d["offset"].to(DEV), d["mask"].to(DEV), b, cin, h,
                           w, ho, wo, k, k, p, p, s, s, dl, dl, dg, col)
    torch.cuda.synchronize()
    ref = od.im2col_nchw(d["x"].double(), d["offset"].double(), d["mask"].double(), k, k, p, p,
                         s, s, dl, dl, dg)
    check(col.cpu(), ref, dtype, f"{entry} {geom}")


# ---------------------------------------------------------------------------------------
# NHWC columns (ext.modulated_deformable_im2col_nhwc_cuda), 2T and raw-y (3T) forms
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("fused_y", [False, True], ids=["2T", "3T"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16, torch.float64],
                         ids=["fp32", "fp16", "bf16", "fp64"])
@pytest.mark.parametrize("geom", [
    (2, 16, 9, 11, 1, 1, 1), (1, 24, 8, 13, 2, 1, 1), (1, 256, 12, 10, 1, 1, 1),
    (2, 5, 7, 6, 1, 1, 1), (1, 40, 10, 9, 1, 2, 2),
])
def test_im2col_nhwc(fused_y, dtype, geom):
    b, cin, h, w, s, p, dl = geom
    d = inputs.nchw_to_nhwc(_rand_problem(b, cin, 4, h, w, 3, s, p, dl, dtype=dtype,
                                          seed=sum(geom) + fused_y))
    ho, wo = od.out_size(h, p, dl, 3, s), od.out_size(w, p, dl, 3, s)
    x = d["x"]
    if fused_y:
        raw = torch.randn(b, ho, wo, 9, generator=torch.Generator().manual_seed(1)).to(dtype)
        y = torch.cat([d["offset"], raw], -1).contiguous()
        off_ref, mask_ref = od.split_y_nhwc(y.double(), 9)
        off_arg, mask_arg = y, y
    else:
        off_ref, mask_ref = d["offset"].double(), d["mask"].double()
        off_arg, mask_arg = d["offset"], d["mask"]
    col = torch.full((b * ho * wo, 9 * cin), float("nan"), dtype=dtype, device=DEV)
    _ext().modulated_deformable_im2col_nhwc_cuda(
        x.to(DEV), off_arg.to(DEV), mask_arg.to(DEV), b, cin, h, w, ho, wo, 3, 3, p, p, s, s,
        dl, dl, 1, col)
    torch.cuda.synchronize()
    ref = od.columns_nhwc(x.double(), off_ref, mask_ref, 3, 3, s, s, p, p, dl, dl)
    check(col.cpu(), ref, dtype, f"nhwc cols {geom}")


# ---------------------------------------------------------------------------------------
# Fused NHWC implicit GEMM (fused_tl.fused_dcn_forward_nhwc -> ext.dcn_fused_fwd_nhwc)
# ---------------------------------------------------------------------------------------

def _cols_dtype(dtype):
    """The kernels round the deformable taps to the input dtype before the matrix cores,
    as the reference's column buffer / A tile does; the oracle does the same."""
    return None if dtype == torch.float32 else dtype


def _fused_ref(d, dtype):
    return od.forward_nhwc(d["x"].double(), d["offset"].double(), d["mask"].double(),
                           d["weight"].double(), d["bias"].double(), d["stride"], d["padding"],
                           d["dilation"], col_dtype=_cols_dtype(dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16],
                         ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("geom", [
    # b, cin, cout, h, w, stride, pad, dil
    (2, 16, 32, 9, 11, 1, 1, 1),
    (1, 64, 64, 32, 32, 1, 1, 1),
    (2, 32, 40, 13, 7, 1, 1, 1),      # Cout tail
    (1, 24, 300, 10, 9, 2, 1, 1),     # stride 2, Cout > 256
    (1, 128, 96, 6, 20, 1, 2, 2),     # dilation 2
    (3, 8, 8, 5, 5, 1, 1, 1),
])
def test_fused_nhwc(dtype, geom):
    b, cin, cout, h, w, s, p, dl = geom
    from modulated_deform_conv import fused_tl
    d = inputs.nchw_to_nhwc(_rand_problem(b, cin, cout, h, w, 3, s, p, dl, dtype=dtype,
                                          seed=sum(geom)))
    out = fused_tl.fused_dcn_forward_nhwc(d["x"].to(DEV), d["offset"].to(DEV),
                                          d["mask"].to(DEV), d["weight"].to(DEV),
                                          d["bias"].to(DEV), s, p, dl)
    torch.cuda.synchronize()
    check(out.cpu(), _fused_ref(d, dtype), dtype, f"fused {geom}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("cfg", ["dcn_res4", "dcn_res5"])
def test_fused_nhwc_full_size(cfg, dtype):
    d = inputs.nchw_to_nhwc(inputs.dcn_inputs(cfg))
    d = {k: (v.to(dtype) if torch.is_tensor(v) else v) for k, v in d.items()}
    from modulated_deform_conv import fused_tl
    out = fused_tl.fused_dcn_forward_nhwc(d["x"].to(DEV), d["offset"].to(DEV),
                                          d["mask"].to(DEV), d["weight"].to(DEV), None, 1, 1, 1)
    torch.cuda.synchronize()
    out = out.cpu()
    assert torch.isfinite(out.float()).all()
    for b in (0, d["x"].shape[0] - 1):
        sub = {k: (v[b:b + 1] if k in ("x", "offset", "mask") else v) for k, v in d.items()}
        sub["bias"] = None
        ref = od.forward_nhwc(sub["x"].double(), sub["offset"].double(), sub["mask"].double(),
                              sub["weight"].double(), None, 1, 1, 1,
                              col_dtype=_cols_dtype(dtype))
        check(out[b:b + 1], ref, dtype, f"{cfg} image {b}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("geom", [
    # b, cin, cout, h, w, k, stride, pad, dil
    (1, 16, 48, 12, 10, 5, 1, 2, 1),  # 25 taps: the general-K kernel
    (2, 32, 64, 9, 9, 1, 1, 0, 1),    # 1x1: a single tap
    (1, 8, 33, 7, 8, 2, 1, 0, 1),     # even kernel, K = 32, Cout tail of 1
])
def test_fused_nhwc_kernel_sizes(dtype, geom):
    b, cin, cout, h, w, k, s, p, dl = geom
    from modulated_deform_conv import fused_tl
    d = inputs.nchw_to_nhwc(_rand_problem(b, cin, cout, h, w, k, s, p, dl, dtype=dtype,
                                          seed=sum(geom)))
    out = fused_tl.fused_dcn_forward_nhwc(d["x"].to(DEV), d["offset"].to(DEV),
                                          d["mask"].to(DEV), d["weight"].to(DEV),
                                          d["bias"].to(DEV), s, p, dl)
    torch.cuda.synchronize()
    check(out.cpu(), _fused_ref(d, dtype), dtype, f"fused k{k} {geom}")


def _packed_layout_ref(weight, dtype):
    """Packed weight layout of dcn_pack_weight, restated on the host (permutation + zeros)."""
    cout, c, kh, kw = weight.shape
    w_nk = weight.permute(0, 2, 3, 1).reshape(cout, kh * kw * c)     # [n][k], k = t*C + c
    if dtype == torch.float32:
        return w_nk.reshape(-1)
    nb, kb = -(-cout // 32), -(-(kh * kw * c) // 16)
    padded = torch.zeros(nb * 32, kb * 16, dtype=weight.dtype)
    padded[:cout, :w_nk.shape[1]] = w_nk
    # block (n/32, k/16); lane (n%32) + 32*((k%16)/8); 8 consecutive k per lane
    blocks = padded.view(nb, 32, kb, 2, 8).permute(0, 2, 3, 1, 4)     # [nb][kb][half][n][8]
    return blocks.reshape(-1)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("shape", [(40, 24, 3, 3), (256, 256, 3, 3), (7, 8, 1, 1),
                                   (33, 16, 5, 5), (70, 48, 3, 3), (32, 64, 7, 7)])
def test_pack_weight_layout(dtype, shape):
    """Packed layout, bit-exact: 16-bit C % 16 == 0 with <= 25 taps goes through LDS (row
    and column tails: 33 x 16 x 5 x 5, 70 x 48), the rest element by element."""
    g = torch.Generator().manual_seed(sum(shape))
    w = torch.randn(*shape, generator=g).to(dtype)
    packed = _ext().dcn_pack_weight(w.to(DEV))
    torch.cuda.synchronize()
    ref = _packed_layout_ref(w, dtype)
    assert packed.shape == ref.shape
    assert torch.equal(packed.cpu(), ref)                            # bit-exact permutation


def test_packed_weight_follows_updates():
    """The weight is packed on every call: in-place updates (autograd-visible or through
    .data, as EMA swaps and weight syncs do) are seen by the next call."""
    from modulated_deform_conv import ModulatedDeformConv2d
    torch.manual_seed(1)
    mod = ModulatedDeformConv2d(16, 32, 3, padding=1).half().to(DEV)
    x = torch.randn(1, 16, 8, 9).half().to(DEV)
    off = (0.5 * torch.randn(1, 18, 8, 9)).half().to(DEV)
    msk = torch.rand(1, 9, 8, 9).half().to(DEV)
    with torch.no_grad():
        a = mod(x, off, msk)
        mod.weight.mul_(-2.0)
        b = mod(x, off, msk)
        w0 = mod.weight.detach().clone()
        mod.weight.data.copy_(-0.5 * w0)      # no version bump, same storage
        c = mod(x, off, msk)
    torch.cuda.synchronize()
    bias = mod.bias.view(1, -1, 1, 1).float()
    torch.testing.assert_close((b.float() - bias), -2.0 * (a.float() - bias), rtol=2e-3,
                               atol=2e-3)
    torch.testing.assert_close((c.float() - bias), (a.float() - bias), rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_dcn_split_nhwc_half_3t(dtype):
    """Raw 3T offset-conv output straight into the fused half-precision kernel."""
    from modulated_deform_conv import dcn_split_nhwc as dsn
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 11, 13, 64, generator=g).to(dtype)
    w_off = (0.05 * torch.randn(27, 64, 3, 3, generator=g)).to(dtype)
    b_off = (0.3 * torch.randn(27, generator=g)).to(dtype)
    weight = (0.1 * torch.randn(96, 64, 3, 3, generator=g)).to(dtype)
    bias = torch.randn(96, generator=g).to(dtype)
    out = dsn.dcn_split_nhwc(*(t.to(DEV) for t in (x, w_off, b_off, weight, bias)), 1, 1, 1)
    torch.cuda.synchronize()
    # the offset conv is accumulated and kept in fp32 inside the kernel: the oracle's
    # float64 offset conv, not a library convolution rounded to the input dtype
    ref = od.mega_forward_nhwc(x.double(), w_off.double(), b_off.double(), weight.double(),
                               bias.double(), 1, 1, 1, col_dtype=dtype)
    check(out.cpu(), ref, dtype, "split 3T half")


# ---------------------------------------------------------------------------------------
# Fused front end: offset conv + sigmoid + gather (ext.modulated_deformable_fused_im2col_nhwc)
# ---------------------------------------------------------------------------------------

def _front_problem(b, cin, h, w, k, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    T = k * k
    x = torch.randn(b, h, w, cin, generator=g).to(dtype)
    # offset-conv outputs of a few pixels, as a trained offset conv gives
    w_off = (2.0 / (T * cin) ** 0.5 * torch.randn(3 * T, T, cin, generator=g)).to(dtype)
    b_off = torch.randn(3 * T, generator=g)
    return x, w_off, b_off


def _front_run(x, w_off, b_off, k, s, p, dl):
    b, h, w, cin = x.shape
    ho, wo = od.out_size(h, p, dl, k, s), od.out_size(w, p, dl, k, s)
    col = torch.empty(b * ho * wo, k * k * cin, dtype=x.dtype, device=DEV)
    _ext().modulated_deformable_fused_im2col_nhwc_cuda(
        x.to(DEV), w_off.to(DEV), b_off.to(DEV), b, cin, h, w, ho, wo, k, k, p, p, s, s, dl, dl,
        1, col)
    torch.cuda.synchronize()
    return col.cpu()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16],
                         ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("geom", [
    # b, cin, h, w, k, stride, pad, dil
    (2, 32, 11, 13, 3, 1, 1, 1),
    (1, 64, 16, 12, 3, 2, 1, 1),
    (1, 16, 9, 9, 3, 1, 2, 2),
    (1, 8, 6, 7, 1, 1, 0, 1),
])
def test_fused_front_end(dtype, geom):
    b, cin, h, w, k, s, p, dl = geom
    x, w_off, b_off = _front_problem(b, cin, h, w, k, dtype, sum(geom))
    col = _front_run(x, w_off, b_off, k, s, p, dl)
    ref = od.fused_front_end_columns(x.double(), w_off.double(), b_off.double(), k, k, s, p, dl,
                                     col_dtype=_cols_dtype(dtype))
    check(col, ref, dtype, f"front end {geom}")


def test_fused_front_end_fp32_large_kernel():
    x, w_off, b_off = _front_problem(1, 8, 10, 9, 5, torch.float32, 7)
    col = _front_run(x, w_off, b_off, 5, 1, 2, 1)
    ref = od.fused_front_end_columns(x.double(), w_off.double(), b_off.double(), 5, 5, 1, 2, 1)
    check(col, ref, torch.float32, "front end 5x5")


def test_fused_front_end_res4_fp16():
    """BASELINE res4 shape (B=6, 256 channels, 58x100), first and last image vs the oracle."""
    d = inputs.nchw_to_nhwc(inputs.dcn_inputs("dcn_res4"))
    x = d["x"].to(torch.float16)
    _, w_off, b_off = _front_problem(1, 256, 1, 1, 3, torch.float16, 11)
    col = _front_run(x, w_off, b_off, 3, 1, 1, 1).view(6, -1, 9 * 256)
    assert torch.isfinite(col.float()).all()
    for b in (0, 5):
        ref = od.fused_front_end_columns(x[b:b + 1].double(), w_off.double(), b_off.double(), 3,
                                         3, 1, 1, 1, col_dtype=torch.float16)
        check(col[b], ref, torch.float16, f"front end res4 image {b}")


@pytest.mark.parametrize("dtype", HALF, ids=["fp16", "bf16"])
@pytest.mark.parametrize("form", ["mask", "y3t"])
@pytest.mark.parametrize("shape", [
    # batch, cin, cout, h, w (M = b * h * w, stride 1, pad 1)
    (2, 64, 200, 130, 128),   # one column half, 8- and 9-block row ranges, column tail
    (1, 64, 320, 90, 100),    # two column halves (the second 64 wide), 4- and 5-block ranges
    (1, 128, 512, 80, 110),   # two full halves, 4- and 5-block ranges
    (2, 64, 202, 130, 128),   # Cout % 8 != 0: the tiled kernel (16-byte output pieces)
], ids=["half1", "half2-tail", "half2", "cout202"])
def test_fused_half_row_balanced(dtype, form, shape):
    """Shapes that take the row-balanced persistent kernel (on a 256-CU device: NRB - 1 or
    NRB row blocks per workgroup, a partial last row block, one or two 256-column halves
    of Cout). Every output against explicit columns (the NHWC gather kernel, in the input
    dtype as the reference's column buffer) times the weight in fp32 on the GPU; the first
    and last 1500 rows against the float64 oracle."""
    from modulated_deform_conv import fused_tl
    b, cin, cout, h, w = shape
    g = torch.Generator().manual_seed(21)
    x = torch.randn(b, h, w, cin, generator=g).to(dtype)
    off = 2.0 * torch.randn(b, h, w, 18, generator=g)
    off.view(-1)[::13] = 40.0
    weight = (0.1 * torch.randn(cout, cin, 3, 3, generator=g)).to(dtype)
    bias = torch.randn(cout, generator=g).to(dtype)
    if form == "y3t":
        y = torch.cat([off, torch.randn(b, h, w, 9, generator=g)], -1).to(dtype)
        offset, mask = y, None
        off_r, msk_r = od.split_y_nhwc(y.double(), 9)
    else:
        offset = off.to(dtype)
        mask = torch.rand(b, h, w, 9, generator=g).to(dtype)
        off_r, msk_r = offset.double(), mask.double()
    from modulated_deform_conv import dcn_split_nhwc as dsn
    dv = lambda t: None if t is None else t.to(DEV)
    if form == "y3t":
        out = dsn._fused_forward(dv(x), dv(offset), None, dv(weight), dv(bias), 1, 1, 1)
        cols = dsn.gather_cols_nhwc(dv(x), dv(offset), None, 3, 3, 1, 1, 1)
    else:
        out = fused_tl.fused_dcn_forward_nhwc(dv(x), dv(offset), dv(mask), dv(weight),
                                              dv(bias), 1, 1, 1)
        cols = fused_tl.dcn_gather_cols_nhwc(dv(x), dv(offset), dv(mask), 3, 3, 1, 1, 1)
    w_flat = weight.to(DEV).permute(2, 3, 1, 0).reshape(-1, cout).float()
    split = (cols.float() @ w_flat + bias.to(DEV).float()).view(out.shape)
    torch.cuda.synchronize()
    check(out.float().cpu(), split.cpu(), dtype, f"row-balanced {form} vs columns x weight")
    ref = od.forward_nhwc(x.double(), off_r, msk_r, weight.double(), bias.double(), 1, 1, 1,
                          col_dtype=dtype)
    flat_out, flat_ref = out.cpu().reshape(-1, cout), ref.reshape(-1, cout)
    for sl in (slice(0, 1500), slice(-1500, None)):
        check(flat_out[sl], flat_ref[sl], dtype, f"row-balanced {form} vs oracle")


@pytest.mark.parametrize("dtype", HALF, ids=["fp16", "bf16"])
def test_fused_unaligned_output(dtype):
    """A persistent-kernel shape with an output that starts 2 bytes past a 16-byte boundary
    (a contiguous view one element into a larger buffer): the 16-byte stores of the
    persistent kernel's epilogue do not apply, the tiled kernel writes the rows, the result
    matches the aligned call within the dtype's tolerance and the elements around the
    output keep their values."""
    ext = _ext()
    b, cin, cout, h, w = 2, 64, 200, 130, 128
    g = torch.Generator().manual_seed(33)
    x = torch.randn(b, h, w, cin, generator=g).to(dtype).to(DEV)
    off = (2.0 * torch.randn(b, h, w, 18, generator=g)).to(dtype).to(DEV)
    mask = torch.rand(b, h, w, 9, generator=g).to(dtype).to(DEV)
    weight = (0.1 * torch.randn(cout, cin, 3, 3, generator=g)).to(dtype).to(DEV)
    bias = torch.randn(cout, generator=g).to(dtype).to(DEV)
    packed = ext.dcn_pack_weight(weight)
    n = b * h * w * cout
    aligned = torch.empty(b, h, w, cout, dtype=dtype, device=DEV)
    buf = torch.full((n + 16,), 7.0, dtype=dtype, device=DEV)
    shifted = buf[1:1 + n].view(b, h, w, cout)
    assert shifted.data_ptr() % 16 == 2
    for out in (aligned, shifted):
        ext.dcn_fused_fwd_nhwc(x, off, mask, packed, bias, b, cin, h, w, h, w, cout, 3, 3, 1,
                               1, 1, 1, 1, 1, out)
    torch.cuda.synchronize()
    check(shifted.float().cpu(), aligned.float().cpu(), dtype, "unaligned output vs aligned")
    assert buf[0].item() == 7.0 and bool((buf[n + 1:] == 7.0).all())


def test_fused_matches_gather_plus_gemm():
    """Fused kernel == explicit columns (NHWC gather kernel) @ weight, same inputs."""
    d = inputs.nchw_to_nhwc(_rand_problem(2, 64, 128, 20, 24, seed=5, dtype=torch.float32))
    from modulated_deform_conv import fused_tl
    x, off, m, w = (d[k].to(DEV) for k in ("x", "offset", "mask", "weight"))
    fused = fused_tl.fused_dcn_forward_nhwc(x, off, m, w, None, 1, 1, 1)
    cols = fused_tl.dcn_gather_cols_nhwc(x, off, m, 3, 3, 1, 1, 1)
    split = (cols.double() @ w.permute(2, 3, 1, 0).reshape(-1, 128).double()).view_as(fused)
    check(fused.cpu(), split.cpu(), torch.float32, "fused vs split")


# ---------------------------------------------------------------------------------------
# Modules and autograd functions
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("groups,dg", [(1, 1), (2, 1), (1, 2)])
def test_modulated_deform_conv2d_nchw(groups, dg):
    from modulated_deform_conv import modulated_deform_conv2d
    d = _rand_problem(2, 16, 24, 11, 13, dg=dg, groups=groups, seed=groups * 10 + dg)
    out = modulated_deform_conv2d(d["x"].to(DEV), d["offset"].to(DEV), d["mask"].to(DEV),
                                  d["weight"].to(DEV), d["bias"].to(DEV), 1, 1, 1, groups, dg)
    torch.cuda.synchronize()
    ref = od.forward_nchw(d["x"].double(), d["offset"].double(), d["mask"].double(),
                          d["weight"].double(), d["bias"].double(), (1, 1), (1, 1), (1, 1),
                          groups, dg)
    check(out.cpu(), ref, torch.float32, f"nchw module g{groups} dg{dg}")


def test_config1_nchw_fixture():
    """BASELINE configs[0] through the module forward vs the committed fixture."""
    import os
    from modulated_deform_conv import modulated_deform_conv2d
    fx = torch.load(os.path.join(os.path.dirname(__file__), "golden", "dcn_c1.pt"),
                    weights_only=True)
    d = inputs.dcn_inputs("dcn_c1")
    for k, v in fx["checksums"].items():
        assert abs(float(d[k].double().sum() + (d[k].double() ** 2).sum()) - v) < 1e-6 * abs(v)
    out = modulated_deform_conv2d(d["x"].to(DEV), d["offset"].to(DEV), d["mask"].to(DEV),
                                  d["weight"].to(DEV), d["bias"].to(DEV), 1, 1, 1, 1, 1)
    torch.cuda.synchronize()
    check(out.cpu(), fx["out"], torch.float32, "config1")


@pytest.mark.parametrize("cfg", ["dcn_res4", "dcn_res5"])
def test_nchw_fp32_full_size(cfg):
    from modulated_deform_conv import modulated_deform_conv2d
    d = inputs.dcn_inputs(cfg)
    out = modulated_deform_conv2d(d["x"].to(DEV), d["offset"].to(DEV), d["mask"].to(DEV),
                                  d["weight"].to(DEV), None, 1, 1, 1, 1, 1)
    torch.cuda.synchronize()
    out = out.cpu()
    b = d["x"].shape[0] - 1
    ref = od.forward_nchw(d["x"][b:].double(), d["offset"][b:].double(),
                          d["mask"][b:].double(), d["weight"].double(), None, (1, 1), (1, 1),
                          (1, 1))
    check(out[b:], ref, torch.float32, f"{cfg} nchw fp32")


@pytest.mark.parametrize("backend", ["fuse_c", "tilelang", "cuda"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_pack_module(backend, dtype):
    """Pack forward vs the oracle fed with the module's own offset-conv output (the
    offset conv is a library convolution; the check covers the offset/mask split, the
    sigmoid and the deformable kernel)."""
    from modulated_deform_conv import ModulatedDeformConv2dPack
    torch.manual_seed(0)
    mod = ModulatedDeformConv2dPack(32, 48, 3, stride=1, padding=1, backend=backend)
    with torch.no_grad():
        mod.conv_offset.weight.normal_(0, 0.05)
        mod.conv_offset.bias.normal_(0, 0.5)
        mod.bias.normal_()
    mod = mod.to(dtype).to(DEV)
    x = torch.randn(2, 32, 14, 17).to(dtype).to(DEV)
    with torch.no_grad():
        out = mod(x)
        y = mod.conv_offset(x)
    torch.cuda.synchronize()
    off, msk = od.split_y_nchw(y.double().cpu(), 9)
    ref = od.forward_nchw(x.double().cpu(), off, msk, mod.weight.double().cpu(),
                          mod.bias.double().cpu(), (1, 1), (1, 1), (1, 1),
                          col_dtype=_cols_dtype(dtype))
    check(out.cpu(), ref, dtype, f"pack {backend}")


def test_dcn_split_nhwc_bn_relu_epilogue():
    from modulated_deform_conv import dcn_split_nhwc as dsn
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 10, 12, 32, generator=g)
    w_off = 0.05 * torch.randn(27, 32, 3, 3, generator=g)
    b_off = 0.3 * torch.randn(27, generator=g)
    weight = 0.1 * torch.randn(64, 32, 3, 3, generator=g)
    bias = torch.randn(64, generator=g)
    scale = 0.5 + torch.rand(64, generator=g)
    shift = torch.randn(64, generator=g)
    out = dsn.dcn_split_nhwc(*(t.to(DEV) for t in (x, w_off, b_off, weight, bias)), 1, 1, 1,
                             scale.to(DEV), shift.to(DEV), True)
    torch.cuda.synchronize()
    y = F.conv2d(x.double().permute(0, 3, 1, 2), w_off.double(), b_off.double(), 1, 1, 1)
    off, msk = od.split_y_nhwc(y.permute(0, 2, 3, 1), 9)
    conv = od.forward_nhwc(x.double(), off, msk, weight.double(), bias.double(), 1, 1, 1)
    ref = torch.relu(conv * scale.double() + shift.double())
    check(out.cpu(), ref, torch.float32, "bn relu")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16],
                         ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("shape", [(2, 256, 58, 100), (1, 3, 5, 7), (3, 18, 29, 50),
                                   (1, 130, 1, 67)])
def test_transpose_layouts(dtype, shape):
    """The NCHW <-> NHWC layout kernel is a bit-exact copy: tile-aligned, ragged and
    odd-sized shapes (the vector and the scalar path), both directions."""
    import _modulated_deform_conv_ext as ext
    g = torch.Generator().manual_seed(3)
    x = torch.randn(*shape, generator=g).to(dtype).to(DEV)
    y = ext.nchw_to_nhwc(x)
    assert y.shape == (shape[0], shape[2], shape[3], shape[1])
    assert torch.equal(y, x.permute(0, 2, 3, 1).contiguous())
    z = ext.nhwc_to_nchw(y)
    assert torch.equal(z, x)


# ---------------------------------------------------------------------------------------
# Arithmetic of the A operand: one rounding of an fp32 blend
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", HALF, ids=["fp16", "bf16"])
@pytest.mark.parametrize("shape", [(2, 64, 256, 9, 11), (1, 64, 256, 130, 128)],
                         ids=["tiled", "persistent"])
def test_fused_columns_single_rounding(dtype, shape):
    """A selector weight (W[n] = 1 at one k_n, 0 elsewhere) makes every output element one
    element of the deformable A operand, passed exactly through the fp32 MFMA accumulation.
    The kernel blends the four corners in fp32 and rounds once to the input dtype (the
    reference's gather, dcn_fused_nhwc_kernel.cuh:185-187): against the float64 columns
    rounded once (at the kernel's fp32 sampling coordinate), almost all elements are equal (a difference needs the exact value within
    fp32 rounding of a rounding boundary), and each differing one is within one ulp plus
    the fp32 blend's own error (a few 2^-24 of sum |w_q * corner_q|, which shows when the
    corners cancel). A blend in 16-bit arithmetic (weights rounded, partial sums rounded)
    fails both the equality count and the per-element bound."""
    from modulated_deform_conv import fused_tl
    b, cin, cout, h, w = shape
    d = inputs.nchw_to_nhwc(_rand_problem(b, cin, cout, h, w, dtype=dtype, seed=31))
    K = 9 * cin
    sel = (torch.arange(cout) * 37 + 5) % K                  # distinct k per output column
    w_nk = torch.zeros(cout, K)
    w_nk[torch.arange(cout), sel] = 1.0
    weight = w_nk.view(cout, 3, 3, cin).permute(0, 3, 1, 2).contiguous().to(dtype)
    out = fused_tl.fused_dcn_forward_nhwc(d["x"].to(DEV), d["offset"].to(DEV),
                                          d["mask"].to(DEV), weight.to(DEV), None, 1, 1, 1)
    torch.cuda.synchronize()
    got = out.cpu().reshape(-1, cout)
    # the sampling coordinate is an fp32 sum in the kernel, as in the reference's kernels
    cols = od.columns_nhwc(d["x"].double(), d["offset"].double(), d["mask"].double(), 3, 3, 1,
                           1, 1, 1, 1, 1, coord_dtype=torch.float32)
    ref = cols[:, sel].to(dtype)                              # one rounding
    # sum_q |w_q * corner_q|: the columns of |x| (bilinear weights and mask are >= 0)
    mag = od.columns_nhwc(d["x"].double().abs(), d["offset"].double(), d["mask"].double(),
                          3, 3, 1, 1, 1, 1, 1, 1, coord_dtype=torch.float32)[:, sel]
    diff = got != ref
    frac = diff.double().mean().item()
    assert frac < 1e-3, f"{frac:.2e} of the A elements differ from one rounding"
    if diff.any():
        a, r = got[diff].double(), ref[diff].double()
        ulp = (r.abs() * (2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7)).clamp_min(
            2.0 ** -24)
        bound = ulp * 1.0001 + 8 * 2.0 ** -24 * mag[diff]
        far = (a - r).abs() > bound
        assert not far.any(), (
            f"{int(far.sum())} of {a.numel()} differing elements beyond the bound; first "
            f"(got, want): {list(zip(a[far][:6].tolist(), r[far][:6].tolist()))}")


# ---------------------------------------------------------------------------------------
# Offset conv inside: offset_conv_forward_nhwc, the single-kernel forward and its callers
# ---------------------------------------------------------------------------------------

def _mega_problem(b, cin, cout, h, w, dtype, seed, k=3):
    g = torch.Generator().manual_seed(seed)
    T = k * k
    x = torch.randn(b, h, w, cin, generator=g).to(dtype)
    # a trained offset conv gives offsets of a few pixels and mask logits around 0
    w_off = ((1.5 / (T * cin) ** 0.5) * torch.randn(3 * T, cin, k, k, generator=g)).to(dtype)
    b_off = 0.5 * torch.randn(3 * T, generator=g)
    weight = (0.1 * torch.randn(cout, cin, k, k, generator=g)).to(dtype)
    bias = torch.randn(cout, generator=g).to(dtype)
    return x, w_off, b_off, weight, bias


def _mega_ref(x, w_off, b_off, weight, bias, dtype, s=1, p=1, dl=1, relu=False):
    return od.mega_forward_nhwc(x.double(), w_off.double(), b_off.double(), weight.double(),
                                None if bias is None else bias.double(), s, p, dl,
                                col_dtype=_cols_dtype(dtype), relu=relu)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16],
                         ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("geom", [
    # b, cin, h, w, stride, pad, dil
    (2, 64, 9, 11, 1, 1, 1),
    (1, 32, 12, 10, 2, 1, 1),
    (1, 16, 10, 9, 1, 2, 2),
    # half types, 3 x 3 stride 1 with C % 64 == 0: output row segments of one or two
    # subtiles (a 150-pixel row in three segments; no padding); other geometries with
    # C % 64 == 0 take the tiled form (stride 2 with 128-channel steps, dilation 2 with K
    # in two parts adding into y), and C % 64 != 0 with a long K splits by steps
    (1, 256, 12, 10, 1, 1, 1),
    (1, 192, 9, 11, 1, 1, 1),
    (2, 64, 5, 150, 1, 1, 1),
    (1, 128, 8, 40, 1, 0, 1),
    (1, 128, 10, 12, 2, 1, 1),
    (1, 192, 11, 9, 1, 2, 2),
    (1, 136, 10, 9, 1, 1, 1),
])
def test_offset_conv_forward_nhwc(dtype, geom):
    """fused_tl.offset_conv_forward_nhwc: y accumulated and kept in fp32 on the matrix
    cores, offset = y[..., :2T] and mask = sigmoid(y[..., 2T:]) rounded once to the input
    dtype (fused_tl.py:419-470); the fp32 y itself against the float64 conv."""
    from modulated_deform_conv import fused_tl, dcn_split_nhwc as dsn
    b, cin, h, w, s, p, dl = geom
    x, w_off, b_off, _, _ = _mega_problem(b, cin, 8, h, w, dtype, seed=sum(geom))
    off, mask = fused_tl.offset_conv_forward_nhwc(x.to(DEV), w_off.to(DEV), b_off.to(DEV), 3,
                                                  3, s, p, dl)
    y = dsn.offset_conv_y(x.to(DEV), w_off.to(DEV), b_off.to(DEV), s, p, dl)
    torch.cuda.synchronize()
    y_ref = od.offset_conv_nhwc(x.double(), w_off.double(), b_off.double(), s, p, dl)
    check(y.cpu(), y_ref, torch.float32, f"offset conv y {geom}")
    o_ref, m_ref = od.split_y_nhwc(y_ref, 9)
    assert off.dtype == mask.dtype == dtype
    check(off.cpu(), o_ref, dtype, "offset")
    check(mask.cpu(), m_ref, dtype, "mask")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16],
                         ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("shape", [
    # batch, cin, cout, h, w: persistent one-launch shapes on a 256-CU device, then tiled
    (2, 64, 200, 130, 128),   # one column half, 8- and 9-block row ranges, column tail
    (1, 64, 320, 90, 100),    # two column halves, 4- and 5-block ranges
    (2, 32, 48, 11, 13),      # the offset conv, then the fused kernel reading y
], ids=["half1", "half2-tail", "small"])
def test_mega_forward(dtype, shape):
    """fused_tl.fused_dcn_mega_forward_nhwc (fused_tl.py:565-766): offset conv, sigmoid,
    deformable gather and main GEMM in one launch (fp16 / bf16 persistent shapes). Every
    output element against the float64 oracle (offset conv in float64, columns rounded to
    the input dtype as the kernel's A tile), and the fp32 y the kernel writes for the
    backward against the float64 conv."""
    from modulated_deform_conv import fused_tl, dcn_split_nhwc as dsn
    b, cin, cout, h, w = shape
    x, w_off, b_off, weight, bias = _mega_problem(b, cin, cout, h, w, dtype, seed=cin + cout)
    dv = [t.to(DEV) for t in (x, w_off, b_off, weight, bias)]
    out = fused_tl.fused_dcn_mega_forward_nhwc(*dv, 1, 1, 1)
    out2, y = dsn.mega_forward(*dv, 1, 1, 1)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    y_ref = od.offset_conv_nhwc(x.double(), w_off.double(), b_off.double(), 1, 1, 1)
    check(y.cpu(), y_ref, torch.float32, f"mega y {shape}")
    ref = _mega_ref(x, w_off, b_off, weight, bias, dtype)
    check(out.cpu(), ref, dtype, f"mega {shape}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_mega_bn_relu_persistent(dtype):
    """dcn_split_nhwc with the FrozenBN + ReLU epilogue on a one-launch shape: BN folded
    into the packed weight and bias, ReLU in the kernel's store (dcn_split_nhwc.py:178-204)."""
    from modulated_deform_conv import dcn_split_nhwc as dsn
    b, cin, cout, h, w = 2, 64, 200, 130, 128
    x, w_off, b_off, weight, bias = _mega_problem(b, cin, cout, h, w, dtype, seed=9)
    g = torch.Generator().manual_seed(2)
    scale = 0.5 + torch.rand(cout, generator=g)
    shift = torch.randn(cout, generator=g)
    out = dsn.dcn_split_nhwc(*(t.to(DEV) for t in (x, w_off, b_off, weight, bias)), 1, 1, 1,
                             scale.to(DEV), shift.to(DEV), True)
    torch.cuda.synchronize()
    w_eff = (weight.double() * scale.to(dtype).double().view(-1, 1, 1, 1)).to(dtype)
    b_eff = (shift + bias.float() * scale).to(dtype)
    ref = _mega_ref(x, w_off, b_off, w_eff, b_eff, dtype, relu=True)
    assert (out >= 0).all()
    check(out.cpu(), ref, dtype, "mega bn relu")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_full_split_forward_entry_points(dtype):
    """fused_dcn_full_forward_nhwc (offset conv, offsets rounded, fused kernel),
    dcn_forward_split_nhwc and dcn_split_forward_nhwc (one kernel), fused_tl.dcn_split and
    both dcn_apply_nchw adapters against the float64 oracle."""
    from modulated_deform_conv import fused_tl, dcn_split_nhwc as dsn
    x, w_off, b_off, weight, bias = _mega_problem(2, 64, 96, 12, 14, dtype, seed=12)
    dv = [t.to(DEV) for t in (x, w_off, b_off, weight, bias)]
    ref = _mega_ref(x, w_off, b_off, weight, bias, dtype)
    for name, fn in (("full", fused_tl.fused_dcn_full_forward_nhwc),
                     ("split", fused_tl.dcn_forward_split_nhwc),
                     ("split_forward", dsn.dcn_split_forward_nhwc),
                     ("dcn_split", fused_tl.dcn_split)):
        out = fn(*dv, 1, 1, 1)
        torch.cuda.synchronize()
        check(out.detach().cpu(), ref, dtype, name)
    x_nchw = dv[0].permute(0, 3, 1, 2).contiguous()
    for name, fn in (("tl nchw", fused_tl.dcn_apply_nchw), ("fuse_c nchw", dsn.dcn_apply_nchw)):
        out = fn(x_nchw, *dv[1:], 1, 1, 1)
        torch.cuda.synchronize()
        assert out.is_contiguous()
        check(out.detach().permute(0, 2, 3, 1).cpu(), ref, dtype, name)


def test_pack_cuda_channels_last(monkeypatch):
    """Pack(backend='cuda') with ENABLE_CHANNEL_LAST (modulated_deform_conv.py:614-621): the
    NCHW path on contiguous copies, output in channels_last memory format, same values."""
    from modulated_deform_conv import ModulatedDeformConv2dPack
    torch.manual_seed(4)
    mod = ModulatedDeformConv2dPack(32, 40, 3, stride=1, padding=1, backend="cuda")
    with torch.no_grad():
        mod.conv_offset.weight.normal_(0, 0.05)
        mod.conv_offset.bias.normal_(0, 0.5)
    mod = mod.to(DEV)
    x = torch.randn(2, 32, 11, 13).to(DEV).to(memory_format=torch.channels_last)
    with torch.no_grad():
        monkeypatch.setenv("ENABLE_CHANNEL_LAST", "1")
        out_cl = mod(x)
        monkeypatch.setenv("ENABLE_CHANNEL_LAST", "0")
        out = mod(x)
        y = mod.conv_offset(x)
    torch.cuda.synchronize()
    assert out_cl.is_contiguous(memory_format=torch.channels_last)
    off, msk = od.split_y_nchw(y.double().cpu(), 9)
    ref = od.forward_nchw(x.double().cpu(), off, msk, mod.weight.double().cpu(),
                          mod.bias.double().cpu(), (1, 1), (1, 1), (1, 1))
    check(out_cl.cpu(), ref, torch.float32, "channels_last")
    check(out.cpu(), ref, torch.float32, "contiguous")


# ---------------------------------------------------------------------------------------
# Non-finite input: the reference's corner read rule (modulated_deform_conv.py:184-213,
# dcn_fused_nhwc_kernel.cuh:270-301): an in-bounds corner is read whatever its bilinear
# weight (0 * NaN = NaN), an out-of-bounds corner contributes exactly 0.
# ---------------------------------------------------------------------------------------

def _poison_nhwc(x, off, seed):
    """x [B, H, W, C], off [B, Ho, Wo, 18] (stride 1, pad 1, dilation 1, 3 x 3), in place:
      * output pixel (1, 2) of image 0: every tap lands exactly on input pixel (1, 2), whose
        corner of weight 1 is finite and whose weight-0 corners include NaN pixel (2, 3)
        -> the whole output row is NaN;
      * output pixel (Ho - 2, 1) of image 0: every tap far outside (offset +40), and NaN at
        input pixel (H - 1, W - 1), where a clamped read would land -> output = bias;
      * a few random pixels of every image hold NaN or +Inf in all channels."""
    g = torch.Generator().manual_seed(seed)
    B, H, W, C = x.shape
    for b in range(B):
        ys = torch.randint(0, H, (4,), generator=g)
        xs = torch.randint(0, W, (4,), generator=g)
        for k in range(4):
            x[b, ys[k], xs[k], :] = float("nan") if k < 2 else float("inf")
    for (py, px) in ((1, 2), (1, 3), (2, 2)):
        x[0, py, px, :] = 1.0
    x[0, 2, 3, :] = float("nan")
    for t in range(9):
        ki, kj = t // 3, t % 3
        off[0, 1, 2, 2 * t] = 1 - ki        # h_im = 1 - 1 + ki + (1 - ki) = 1
        off[0, 1, 2, 2 * t + 1] = 1 - kj    # w_im = 2 - 1 + kj + (1 - kj) = 2
    x[0, H - 1, W - 1, :] = float("nan")
    off[0, -2, 1, :] = 40.0


def _nonfinite_check(out, ref, dtype, what):
    out, ref = out.double().cpu(), ref.double().cpu()
    assert torch.equal(torch.isnan(out), torch.isnan(ref)), f"{what}: NaN pattern"
    assert torch.equal(torch.isinf(out), torch.isinf(ref)), f"{what}: Inf pattern"
    assert torch.equal(out[torch.isinf(ref)], ref[torch.isinf(ref)]), f"{what}: Inf sign"
    fin = torch.isfinite(ref)
    check(out[fin], ref[fin], dtype, what)
    assert 0.05 < fin.double().mean().item() < 0.999, f"{what}: degenerate poison pattern"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16],
                         ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("shape", [(2, 16, 32, 9, 11), (1, 64, 320, 90, 100)],
                         ids=["tiled", "persistent"])
def test_nonfinite_input_nhwc(shape, dtype):
    """NaN / Inf in x give NaN / Inf exactly where the float64 oracle does (fused NHWC
    forward: the tiled kernel, and in 16-bit types the persistent kernel with two column
    halves), and every finite output matches it to tolerance."""
    from modulated_deform_conv import fused_tl
    b, cin, cout, h, w = shape
    g = torch.Generator().manual_seed(41)
    x = torch.randn(b, h, w, cin, generator=g)
    off = 2.0 * torch.randn(b, h, w, 18, generator=g)
    mask = torch.rand(b, h, w, 9, generator=g)
    weight = 0.1 * torch.randn(cout, cin, 3, 3, generator=g)
    bias = torch.randn(cout, generator=g)
    _poison_nhwc(x, off, seed=42)
    x, off, mask, weight, bias = (t.to(dtype) for t in (x, off, mask, weight, bias))
    out = fused_tl.fused_dcn_forward_nhwc(x.to(DEV), off.to(DEV), mask.to(DEV),
                                          weight.to(DEV), bias.to(DEV), 1, 1, 1)
    torch.cuda.synchronize()
    ref = od.forward_nhwc(x.double(), off.double(), mask.double(), weight.double(),
                          bias.double(), 1, 1, 1, col_dtype=_cols_dtype(dtype))
    what = f"nonfinite nhwc {shape} {dtype}"
    _nonfinite_check(out, ref, dtype, what)
    out = out.cpu()
    assert torch.isnan(out[0, 1, 2].float()).all(), f"{what}: zero-weight NaN corner not read"
    assert torch.equal(out[0, -2, 1], bias), f"{what}: out-of-range taps not exactly 0"


@pytest.mark.parametrize("groups", [1, 2])
def test_nonfinite_input_nchw(groups):
    """The NCHW module forward (groups 1: NHWC fused kernel between transposes; groups 2:
    NCHW column kernel + per-group GEMM) with NaN / Inf in x, against the float64 oracle."""
    from modulated_deform_conv import modulated_deform_conv2d
    g = torch.Generator().manual_seed(43)
    b, cin, cout, h, w = 2, 16, 24, 11, 13
    x = torch.randn(b, h, w, cin, generator=g)
    off = 2.0 * torch.randn(b, h, w, 18, generator=g)
    _poison_nhwc(x, off, seed=44)
    x = x.permute(0, 3, 1, 2).contiguous()
    off = off.permute(0, 3, 1, 2).contiguous()
    mask = torch.rand(b, 9, h, w, generator=g)
    weight = 0.1 * torch.randn(cout, cin // groups, 3, 3, generator=g)
    bias = torch.randn(cout, generator=g)
    out = modulated_deform_conv2d(x.to(DEV), off.to(DEV), mask.to(DEV), weight.to(DEV),
                                  bias.to(DEV), 1, 1, 1, groups, 1)
    torch.cuda.synchronize()
    ref = od.forward_nchw(x.double(), off.double(), mask.double(), weight.double(),
                          bias.double(), (1, 1), (1, 1), (1, 1), groups, 1)
    what = f"nonfinite nchw groups {groups}"
    _nonfinite_check(out, ref, torch.float32, what)
    out = out.cpu()
    if groups == 1:
        assert torch.isnan(out[0, :, 1, 2]).all(), f"{what}: zero-weight NaN corner not read"
    assert torch.equal(out[0, :, -2, 1], bias), f"{what}: out-of-range taps not exactly 0"
