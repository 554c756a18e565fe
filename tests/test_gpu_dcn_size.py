"""The one-launch DCN forward and its callers at the benchmarked sizes, where the K loop
is long and (res5) Cout spans two 256-column halves:

  * res4: B = 6, C = Cout = 256, 58 x 100 (36 K steps of 64 channels per pass);
  * res5: B = 6, C = Cout = 512, 29 x 50 (72 K steps; the two column halves each run the
    offset-conv pass and write y).

fused_dcn_mega_forward_nhwc (fused_tl.py:565-766), dcn_split_nhwc with the FrozenBN +
ReLU epilogue (dcn_split_nhwc.py:178-204) and ModulatedDeformConv2dPack(backend='fuse_c')
on a 256-channel layer are run on the whole batch; the first and the last image are
compared element by element with the float64 oracle (offset conv in float64, deformable
taps rounded to the input dtype as the kernel's A tile, sum in float64), and the fp32 y
the kernel writes for the backward with the float64 offset conv of the whole batch."""
import pytest
import torch

from _tol import check
from oracle import dcn as od

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")

SHAPES = {"res4": (6, 256, 256, 58, 100), "res5": (6, 512, 512, 29, 50)}
IMAGES = [0, 5]


def _problem(b, cin, cout, h, w, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, h, w, cin, generator=g).to(dtype)
    # a trained offset conv gives offsets of a few pixels and mask logits around 0
    w_off = ((1.5 / (9 * cin) ** 0.5) * torch.randn(27, cin, 3, 3, generator=g)).to(dtype)
    b_off = 0.5 * torch.randn(27, generator=g)
    weight = ((1.0 / (9 * cin) ** 0.5) * torch.randn(cout, cin, 3, 3, generator=g)).to(dtype)
    bias = (0.1 * torch.randn(cout, generator=g)).to(dtype)
    return x, w_off, b_off, weight, bias


def _ref(x, w_off, b_off, weight, bias, dtype, relu=False):
    return od.mega_forward_nhwc(x[IMAGES].double(), w_off.double(), b_off.double(),
                                weight.double(), None if bias is None else bias.double(),
                                1, 1, 1, col_dtype=dtype, relu=relu)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("cfg", ["res4", "res5"])
def test_mega_forward_full_size(cfg, dtype):
    from modulated_deform_conv import dcn_split_nhwc as dsn
    from modulated_deform_conv import fused_tl
    x, w_off, b_off, weight, bias = _problem(*SHAPES[cfg], dtype, seed=31)
    dv = [t.to(DEV) for t in (x, w_off, b_off, weight, bias)]
    out = fused_tl.fused_dcn_mega_forward_nhwc(*dv, 1, 1, 1)
    out2, y = dsn.mega_forward(*dv, 1, 1, 1)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    y_ref = od.offset_conv_nhwc(x.double(), w_off.double(), b_off.double(), 1, 1, 1)
    check(y.cpu(), y_ref, torch.float32, f"{cfg} {dtype} y")
    check(out[IMAGES].cpu(), _ref(x, w_off, b_off, weight, bias, dtype), dtype,
          f"{cfg} {dtype} one launch")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("cfg", ["res4", "res5"])
def test_split_bn_relu_full_size(cfg, dtype):
    """dcn_split_nhwc: FrozenBN folded into the packed weight and bias, ReLU in the store."""
    from modulated_deform_conv import dcn_split_nhwc as dsn
    b, cin, cout, h, w = SHAPES[cfg]
    x, w_off, b_off, weight, bias = _problem(b, cin, cout, h, w, dtype, seed=37)
    g = torch.Generator().manual_seed(5)
    scale = 0.5 + torch.rand(cout, generator=g)
    shift = 0.2 * torch.randn(cout, generator=g)
    out = dsn.dcn_split_nhwc(*(t.to(DEV) for t in (x, w_off, b_off, weight, bias)), 1, 1, 1,
                             scale.to(DEV), shift.to(DEV), True)
    torch.cuda.synchronize()
    assert (out >= 0).all()
    w_eff = (weight.double() * scale.to(dtype).double().view(-1, 1, 1, 1)).to(dtype)
    b_eff = (shift + bias.float() * scale).to(dtype)
    check(out[IMAGES].cpu(), _ref(x, w_off, b_off, w_eff, b_eff, dtype, relu=True), dtype,
          f"{cfg} {dtype} bn relu")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_pack_fuse_c_256_channels(dtype):
    """ModulatedDeformConv2dPack(backend='fuse_c') on a res4 layer (NCHW in and out)."""
    from modulated_deform_conv import ModulatedDeformConv2dPack
    torch.manual_seed(41)
    mod = ModulatedDeformConv2dPack(256, 256, 3, stride=1, padding=1, backend="fuse_c")
    with torch.no_grad():
        mod.conv_offset.weight.normal_(0, 1.5 / (9 * 256) ** 0.5)
        mod.conv_offset.bias.normal_(0, 0.5)
        mod.weight.normal_(0, 1.0 / (9 * 256) ** 0.5)
        mod.bias.normal_(0, 0.1)
    mod = mod.to(dtype).to(DEV)
    x = torch.randn(6, 256, 58, 100).to(dtype)
    with torch.no_grad():
        out = mod(x.to(DEV))
    torch.cuda.synchronize()
    x_nhwc = x.permute(0, 2, 3, 1)
    ref = _ref(x_nhwc, mod.conv_offset.weight.cpu(), mod.conv_offset.bias.float().cpu(),
               mod.weight.cpu(), mod.bias.cpu(), dtype)
    check(out[IMAGES].permute(0, 2, 3, 1).cpu(), ref, dtype, f"pack fuse_c {dtype}")


# Shapes off the B = 6 benchmark: (batch, C, Cout, H, W). On a 256-CU device: B=1 res4
# (363 row blocks, chunks of 1-2 blocks, 80-row tiles), B=4 res4 (1450 blocks, chunks of
# 5-6, 144-row tiles), B=8 res4 (2900 blocks: two chunks per workgroup), B=1 res5 (two
# column halves, 91 blocks: most chunks of one block, some workgroups idle), a 2 x 9 x 7
# map (most chunks empty) and an odd width with Cout 320.
GENERAL = [(1, 256, 256, 58, 100), (4, 256, 256, 58, 100), (8, 256, 256, 58, 100),
           (1, 512, 512, 29, 50), (2, 64, 192, 9, 7), (3, 128, 320, 37, 61)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("shape", GENERAL, ids=lambda s: "x".join(map(str, s)))
def test_persistent_schedule_any_rows(shape, dtype):
    """The chunked persistent schedule at row counts off the benchmark bands: the fused
    forward (offsets and mask given) and the one-launch forward, every pixel against the
    float64 oracle (images 0 and last for the large batches)."""
    from modulated_deform_conv import fused_tl
    b, cin, cout, h, w = shape
    x, w_off, b_off, weight, bias = _problem(b, cin, cout, h, w, dtype, seed=sum(shape))
    imgs = [0, b - 1] if b > 2 else list(range(b))
    dv = [t.to(DEV) for t in (x, w_off, b_off, weight, bias)]
    out = fused_tl.fused_dcn_mega_forward_nhwc(*dv, 1, 1, 1)
    torch.cuda.synchronize()
    ref = od.mega_forward_nhwc(x[imgs].double(), w_off.double(), b_off.double(),
                               weight.double(), bias.double(), 1, 1, 1, col_dtype=dtype)
    check(out[imgs].cpu(), ref, dtype, f"one launch {shape}")
    # fused kernel with offsets and mask from the float64 offset conv, rounded to dtype
    y = od.offset_conv_nhwc(x.double(), w_off.double(), b_off.double(), 1, 1, 1)
    off, msk = od.split_y_nhwc(y, 9)
    off, msk = off.to(dtype), msk.to(dtype)
    out = fused_tl.fused_dcn_forward_nhwc(x.to(DEV), off.to(DEV), msk.to(DEV), weight.to(DEV),
                                          bias.to(DEV), 1, 1, 1)
    torch.cuda.synchronize()
    ref = od.forward_nhwc(x[imgs].double(), off[imgs].double(), msk[imgs].double(),
                          weight.double(), bias.double(), 1, 1, 1, col_dtype=dtype,
                          coord_dtype=torch.float32)
    check(out[imgs].cpu(), ref, dtype, f"fused {shape}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_empty_batch(dtype):
    """A batch of 0 images: every forward entry point returns empty outputs of the right
    shapes without launching (the C ABI returns before any kernel for zero rows)."""
    from modulated_deform_conv import fused_tl, dcn_split_nhwc as dsn
    x, w_off, b_off, weight, bias = _problem(0, 64, 192, 9, 7, dtype, seed=3)
    dv = [t.to(DEV) for t in (x, w_off, b_off, weight, bias)]
    out = fused_tl.fused_dcn_mega_forward_nhwc(*dv, 1, 1, 1)
    out2, y = dsn.mega_forward(*dv, 1, 1, 1)
    off, msk = fused_tl.offset_conv_forward_nhwc(dv[0], dv[1], dv[2], 3, 3, 1, 1, 1)
    out3 = fused_tl.fused_dcn_forward_nhwc(dv[0], off, msk, dv[3], dv[4], 1, 1, 1)
    torch.cuda.synchronize()
    assert out.shape == out2.shape == out3.shape == (0, 9, 7, 192)
    assert y.shape == (0, 9, 7, 27) and off.shape == (0, 9, 7, 18) and msk.shape == (0, 9, 7, 9)
