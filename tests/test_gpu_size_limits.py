"""Behaviour at the 32-bit buffer-offset limit. The fast kernels address one batch of MSDA
value (one image of DCN input) through a buffer descriptor with a 32-bit range:
  * MSDA forward: a batch of value of 2 GiB or more takes msda_generic_kernel (64-bit
    indexing) and must still match the oracle, including samples past byte offset 2^31;
  * DCN fused NHWC forward: the whole input goes through one descriptor, so an input over
    2 GiB is rejected with an error before any launch (the reference's own NHWC gather
    stops earlier, at an int32 column element count, dcn_fused_nhwc_cuda.cu:37-40)."""
import pytest
import torch

from _tol import check
from oracle import msda as om

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def test_msda_forward_batch_over_2gib():
    """One level of 4100 x 4100 positions, one head of 32 fp32 channels: 2.15 GB of value
    per batch. Uniform samples put about half the corners past byte offset 2^31."""
    import msda_opt2
    H = W = 4100
    g = torch.Generator(device=DEV).manual_seed(51)
    value = torch.randn(1, H * W, 1, 32, generator=g, device=DEV)
    assert value.numel() * 4 >= 1 << 31
    nq, P = 64, 4
    gc = torch.Generator().manual_seed(52)
    loc = torch.rand(1, nq, 1, 1, P, 2, generator=gc)
    loc[0, 0, 0, 0, :, :] = torch.tensor([1.0 - 0.5 / W, 1.0 - 0.5 / H])  # near the last pixel
    attn = torch.softmax(torch.randn(1, nq, 1, P, generator=gc), -1).view(1, nq, 1, 1, P)
    shapes = torch.tensor([[H, W]], dtype=torch.int64)
    lsi = torch.tensor([0], dtype=torch.int64)
    out = msda_opt2.ms_deform_attn_forward(value, shapes.to(DEV), lsi.to(DEV), loc.to(DEV),
                                           attn.to(DEV))
    torch.cuda.synchronize()
    # fp32 sampling coordinates, as the kernels (one ulp of 4100 is 4.9e-4)
    ref = om.forward(value.cpu().double(), shapes, lsi, loc.double(), attn.double(),
                     coord_dtype=torch.float32)
    check(out.cpu(), ref, torch.float32, "msda batch over 2 GiB")


def test_dcn_input_over_2gib_rejected():
    """A 2100 x 2100 x 256 fp16 input (2.26 GB) through the fused NHWC forward: a clear
    error, no launch."""
    from modulated_deform_conv import fused_tl
    H = W = 2100
    C = Cout = 256
    x = torch.empty(1, H, W, C, dtype=torch.float16, device=DEV)
    off = torch.zeros(1, H, W, 18, dtype=torch.float16, device=DEV)
    mask = torch.ones(1, H, W, 9, dtype=torch.float16, device=DEV)
    weight = torch.zeros(Cout, C, 3, 3, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="too large for 32-bit buffer offsets"):
        fused_tl.fused_dcn_forward_nhwc(x, off, mask, weight, None, 1, 1, 1)
