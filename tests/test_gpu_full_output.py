"""Whole-output parity at the BASELINE sizes: every element is compared, not a sample.

  * MSDA forward, SCA / TSA / DETR, every query: the specialised kernels against the
    generic one-thread-per-output kernel (force_generic=True), an independent
    implementation of the same arithmetic.
  * DCN res4 / res5 fused forward, fp16 / bf16 / fp32, all six images: against the float64
    oracle (taps rounded to the input dtype as the kernel's A tile, sum in float64, at the
    fp32 sampling coordinates the kernels and the reference's kernels use).
  * DCN NHWC column-to-image backward at res4 / res5, one whole image: against autograd of
    the float64 oracle columns.
  * MSDA backward, one whole SCA camera: all three gradients against the oracle.

fp32 comparisons of two fp32 implementations use twice the fp32 bound (each is within the
bound of the exact value); comparisons against the oracle use tests/_tol.py as is."""
import pytest
import torch

from _tol import check
from oracle import dcn as od
from oracle import inputs
from oracle import msda as om

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _check_two_fp32(a, r, what):
    a, r = a.double().cpu(), r.double().cpu()
    err = (a - r).abs()
    bad = err > 2e-4 + 2e-4 * r.abs()
    assert not bad.any(), (f"{what}: {int(bad.sum())}/{a.numel()} outside 2e-4 abs+rel, max "
                           f"err {err.max().item():.3e}")


def _msda_dev(d, dtype):
    return dict(value=d["value"].to(dtype).to(DEV), spatial_shapes=d["spatial_shapes"].to(DEV),
                level_start_index=d["level_start_index"].to(DEV),
                sampling_loc=d["sampling_loc"].to(dtype).to(DEV),
                attn_weight=d["attn_weight"].to(dtype).to(DEV))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16],
                         ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("cfg", ["msda_sca", "msda_tsa", "msda_detr"])
def test_msda_forward_every_query(cfg, dtype):
    import msda_opt2
    d = inputs.msda_inputs(cfg)
    dd = _msda_dev(d, dtype)
    fast = msda_opt2.ms_deform_attn_forward(**dd)
    generic = msda_opt2.ms_deform_attn_forward(**dd, force_generic=True)
    torch.cuda.synchronize()
    assert fast.shape == generic.shape and fast.dtype == dtype
    if dtype == torch.float32:
        _check_two_fp32(fast, generic, f"{cfg} every query")
    else:
        check(fast.cpu(), generic.double().cpu(), dtype, f"{cfg} {dtype} every query")


def _cols_dtype(dtype):
    return None if dtype == torch.float32 else dtype


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("cfg", ["dcn_res4", "dcn_res5"])
def test_dcn_fused_every_pixel(cfg, dtype):
    """All six images of the fused forward against the float64 oracle."""
    from modulated_deform_conv import fused_tl
    d = inputs.nchw_to_nhwc(inputs.dcn_inputs(cfg))
    d = {k: (v.to(dtype) if torch.is_tensor(v) else v) for k, v in d.items()}
    out = fused_tl.fused_dcn_forward_nhwc(d["x"].to(DEV), d["offset"].to(DEV),
                                          d["mask"].to(DEV), d["weight"].to(DEV), None, 1, 1, 1)
    torch.cuda.synchronize()
    ref = od.forward_nhwc(d["x"].double(), d["offset"].double(), d["mask"].double(),
                          d["weight"].double(), None, 1, 1, 1, col_dtype=_cols_dtype(dtype),
                          coord_dtype=torch.float32)
    check(out.cpu(), ref, dtype, f"{cfg} {dtype} every pixel")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("cfg", ["dcn_res4", "dcn_res5"])
def test_dcn_col2im_nhwc_whole_image(cfg, dtype):
    """grad_x (binned kernel), grad_offset and grad_mask of one full-size image."""
    import _modulated_deform_conv_ext as ext
    d = inputs.nchw_to_nhwc(inputs.dcn_inputs(cfg, batch=1))
    x, off, msk = (d[k].to(dtype) for k in ("x", "offset", "mask"))
    b, h, w, c = x.shape
    g = torch.Generator().manual_seed(23)
    dcol = torch.randn(b * h * w, 9 * c, generator=g).to(dtype)
    gx = torch.zeros(b, h, w, c, device=DEV)
    goff = torch.empty(b, h, w, 18, device=DEV)
    gmask = torch.empty(b, h, w, 9, device=DEV)
    ext.modulated_deformable_col2im_nhwc_cuda(dcol.to(DEV), x.to(DEV), off.to(DEV), msk.to(DEV),
                                              b, c, h, w, h, w, 3, 3, 1, 1, 1, 1, 1, 1, 1, gx,
                                              goff, gmask)
    torch.cuda.synchronize()
    leaves = [t.double().requires_grad_() for t in (x, off, msk)]
    # at the kernel's fp32 sampling coordinates: a coordinate that rounds across a cell
    # edge moves the sample into the next cell, where the bilinear derivative differs
    cols = od.columns_nhwc(*leaves, 3, 3, 1, 1, 1, 1, 1, 1, gate=False,
                           coord_dtype=torch.float32)
    grads = torch.autograd.grad((cols * dcol.double()).sum(), leaves)
    tol = torch.float32 if dtype == torch.float32 else dtype
    for name, a, r in zip(("grad_x", "grad_offset", "grad_mask"), (gx, goff, gmask), grads):
        check(a.cpu(), r, tol, f"{cfg} {dtype} whole image {name}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_msda_backward_one_camera_whole(dtype):
    """One SCA camera (Len_in 30825, 10000 queries, 8 heads, 4 levels x 8 points): every
    element of grad_value, grad_sampling_loc and grad_attn_weight against the oracle."""
    import msda_opt2
    d = inputs.msda_inputs("msda_sca", batch=1)
    g = torch.Generator().manual_seed(11)
    go = torch.randn(1, d["sampling_loc"].shape[1], 256, generator=g).to(dtype)
    dd = _msda_dev(d, dtype)
    got = msda_opt2.ms_deform_attn_backward(**dd, grad_output=go.to(DEV))
    torch.cuda.synchronize()
    ref = om.backward(d["value"].to(dtype).double(), d["spatial_shapes"],
                      d["level_start_index"], d["sampling_loc"].to(dtype).double(),
                      d["attn_weight"].to(dtype).double(), go.double(),
                      coord_dtype=torch.float32)
    for name, a, r in zip(("grad_value", "grad_sampling_loc", "grad_attn_weight"), got, ref):
        check(a.cpu(), r, dtype, f"SCA camera {dtype} {name}")
