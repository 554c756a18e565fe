"""The allocation-free fused front end (bevk_modulated_deformable_fused_im2col_nhwc_noalloc)
against the workspace entry point it mirrors (bevk_modulated_deformable_fused_im2col_nhwc):
same kernels, so the columns must be bit-identical; two calls in a row, the second with a
smaller input (the library's static scratch keeps the first call's contents); the call
captured in a HIP graph and replayed, with eager work between the replays, bit-identical
to the eager call every time; a shape whose scratch need exceeds the static scratch is
rejected before any device work."""
import pytest
import torch

import _bevk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _problem(b, c, h, w, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, h, w, c, generator=g).to(dtype).to(DEV)
    w_off = (2.0 / (9 * c) ** 0.5 * torch.randn(27, 9, c, generator=g)).to(dtype).to(DEV)
    b_off = torch.randn(27, generator=g).to(DEV)
    return x, w_off, b_off


def _run_noalloc(x, w_off, b_off, col):
    b, h, w, c = x.shape
    _bevk.call("bevk_modulated_deformable_fused_im2col_nhwc_noalloc", _bevk.dtype_code(x),
               _bevk.ptr(x), _bevk.ptr(w_off), _bevk.ptr(b_off), b, c, h, w, h, w, 3, 3, 1, 1,
               1, 1, 1, 1, 1, _bevk.ptr(col), _bevk.stream_of(x))


def _run_workspace(x, w_off, b_off):
    import _modulated_deform_conv_ext as ext
    b, h, w, c = x.shape
    col = torch.empty(b * h * w, 9 * c, dtype=x.dtype, device=DEV)
    ext.modulated_deformable_fused_im2col_nhwc_cuda(x, w_off, b_off, b, c, h, w, h, w, 3, 3, 1,
                                                    1, 1, 1, 1, 1, 1, col)
    return col


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["fp16", "bf16", "fp32"])
def test_noalloc_matches_workspace_entry(dtype):
    for (b, c, h, w), seed in (((2, 64, 30, 41), 1), ((1, 32, 13, 17), 2)):
        x, w_off, b_off = _problem(b, c, h, w, dtype, seed)
        col = torch.full((b * h * w, 9 * c), float("nan"), dtype=dtype, device=DEV)
        _run_noalloc(x, w_off, b_off, col)
        ref = _run_workspace(x, w_off, b_off)
        torch.cuda.synchronize()
        assert torch.isfinite(col.float()).all()
        assert torch.equal(col, ref), f"shape {(b, c, h, w)}: noalloc != workspace entry"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["fp16", "bf16", "fp32"])
def test_noalloc_graph_capture(dtype):
    """The entry point allocates nothing, so it can be captured: one eager warm-up call,
    capture on a side stream, then replays (with other inputs copied into the captured
    buffers and eager library calls in between), each compared with the eager result."""
    b, c, h, w = 2, 64, 30, 41
    x, w_off, b_off = _problem(b, c, h, w, dtype, 4)
    col = torch.empty(b * h * w, 9 * c, dtype=dtype, device=DEV)
    _run_noalloc(x, w_off, b_off, col)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            _run_noalloc(x, w_off, b_off, col)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for seed in (5, 6, 7):
        x2, w2, bo2 = _problem(b, c, h, w, dtype, seed)
        x.copy_(x2)
        w_off.copy_(w2)
        b_off.copy_(bo2)
        col.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        ref = _run_workspace(x2, w2, bo2)  # eager, between replays
        torch.cuda.synchronize()
        assert torch.equal(col, ref), f"replay with seed {seed} != eager"


def test_noalloc_rejects_oversize():
    # y alone needs 160000 x 27 x 4 bytes > 16 MiB of static scratch
    x, w_off, b_off = _problem(1, 16, 400, 400, torch.float16, 3)
    col = torch.empty(1, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="static scratch"):
        _run_noalloc(x, w_off, b_off, col)
