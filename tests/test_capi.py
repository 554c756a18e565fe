"""libbevk.so's C ABI on the CPU: the library loads without a GPU, exports every entry
point include/bev_kernels.h declares, and rejects bad arguments (status code + message)
before any device work. No call here reaches a HIP launch."""
import ctypes
import os
import re

import pytest

import _bevk

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "bev_kernels.h")
INVALID, UNSUPPORTED = 1, 2


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bevk_[a-z0-9_]+)\s*\(", text)))


def test_header_matches_binding_table():
    assert declared_symbols() == sorted(_bevk.exported_symbols())


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_bevk.library_path())
    for name in declared_symbols():
        assert hasattr(lib, name), f"{name} missing from {_bevk.library_path()}"


def test_version():
    assert _bevk.version().startswith("bevk ")


def _err():
    return _bevk.lib().bevk_last_error().decode()


NULL = None


def _nchw(entry, dtype=0, **kw):
    a = dict(b=1, c=4, h=5, w=5, ho=5, wo=5, kh=3, kw=3, ph=1, pw=1, sh=1, sw=1, dh=1, dw=1, dg=1)
    a.update(kw)
    return getattr(_bevk.lib(), entry)(
        dtype, NULL, NULL, NULL, a["b"], a["c"], a["h"], a["w"], a["ho"], a["wo"], a["kh"],
        a["kw"], a["ph"], a["pw"], a["sh"], a["sw"], a["dh"], a["dw"], a["dg"], NULL, NULL)


@pytest.mark.parametrize("entry", ["bevk_modulated_deformable_im2col",
                                   "bevk_modulated_deformable_im2col_opt"])
def test_nchw_validation(entry):
    assert _nchw(entry, ho=4) == INVALID and "does not match" in _err()
    assert _nchw(entry, dg=0) == INVALID and "deformable_group" in _err()
    assert _nchw(entry, c=6, dg=4) == INVALID and "divisible" in _err()
    assert _nchw(entry, sh=0) == INVALID
    assert _nchw(entry, dtype=9) == INVALID and "dtype" in _err()
    assert _nchw(entry) == INVALID and "null" in _err()   # valid sizes, no buffers
    assert _nchw(entry, b=0) == 0                          # empty: nothing to do


def _nhwc(dtype=0, last=18, dg=1, c=8, b=1):
    return _bevk.lib().bevk_modulated_deformable_im2col_nhwc(
        dtype, NULL, NULL, last, NULL, b, c, 5, 5, 5, 5, 3, 3, 1, 1, 1, 1, 1, 1, dg, NULL, NULL)


def test_nhwc_validation():
    assert _nhwc(dg=2) == INVALID and "deformable_group == 1" in _err()
    assert _nhwc(last=20) == INVALID and "2T" in _err()
    assert _nhwc() == INVALID and "null" in _err()
    assert _nhwc(last=27) == INVALID and "null" in _err()
    assert _nhwc(b=0) == 0


def _fused(dtype=1, c=16, cout=8, last=18):
    return _bevk.lib().bevk_dcn_fused_fwd_nhwc(
        dtype, NULL, NULL, last, NULL, NULL, NULL, 1, c, 5, 5, 5, 5, cout, 3, 3, 1, 1, 1, 1, 1,
        1, NULL, NULL)


def test_fused_validation():
    assert _fused(dtype=3) == UNSUPPORTED and "Double" in _err()
    assert _fused(c=12) == UNSUPPORTED and "multiple of 8" in _err()     # fp16 needs C % 8
    assert _fused(dtype=0, c=6) == UNSUPPORTED and "multiple of 4" in _err()
    assert _fused(last=21) == INVALID
    assert _fused() == INVALID and "null" in _err()
    assert _fused(cout=0) == 0


def test_packed_weight_bytes():
    f = _bevk.lib().bevk_dcn_packed_weight_bytes
    assert f(0, 256, 3, 3, 256) == 256 * 9 * 256 * 4                # fp32: [Cout][kh][kw][C]
    # half types: whole 32 x 16 fragment blocks of 2-byte elements
    assert f(1, 256, 3, 3, 256) == 8 * 144 * 512 * 2
    assert f(2, 40, 3, 3, 8) == 2 * 5 * 512 * 2                      # K = 72 -> 5 blocks
    assert f(1, 0, 3, 3, 8) == 0
    assert f(3, 8, 3, 3, 8) == -1                                    # no fp64 fused kernel
    assert f(1, 8, 0, 3, 8) == -1


def test_fused_im2col_workspace_bytes():
    f = _bevk.lib().bevk_dcn_fused_im2col_nhwc_workspace_bytes
    packed = 1 * 144 * 512 * 2                                  # 27 -> one 32-column block
    y_off = (packed + 255) // 256 * 256
    assert f(1, 6, 256, 58, 100, 3, 3) == y_off + 6 * 58 * 100 * 27 * 4
    assert f(0, 1, 8, 4, 4, 3, 3) == (27 * 72 * 4 + 255) // 256 * 256 + 16 * 27 * 4
    assert f(3, 1, 8, 4, 4, 3, 3) == -1
    assert f(1, 1, 8, 4, 4, 0, 3) == -1


def _front(dtype=1, c=16, dg=1, kh=3, kw=3, ws=1 << 20, b=1):
    ho = 5 + 2 - kh + 1                                          # pad 1, stride 1, dilation 1
    return _bevk.lib().bevk_modulated_deformable_fused_im2col_nhwc(
        dtype, NULL, NULL, NULL, b, c, 5, 5, ho, ho, kh, kw, 1, 1, 1, 1, 1, 1, dg, NULL, ws,
        NULL, NULL)


def test_fused_im2col_validation():
    assert _front(dg=2) == INVALID and "deformable_group == 1" in _err()
    assert _front(dtype=3) == UNSUPPORTED and "Double" in _err()
    assert _front(kh=5, kw=5) == UNSUPPORTED and "9 taps" in _err()
    assert _front(c=12) == UNSUPPORTED and "multiple of 8" in _err()
    assert _front(ws=16) == INVALID and "workspace" in _err()
    assert _front() == INVALID and "null" in _err()
    assert _front(b=0) == 0


def test_pack_weight_validation():
    f = _bevk.lib().bevk_dcn_pack_weight
    assert f(3, NULL, 8, 3, 3, 8, NULL, NULL) == UNSUPPORTED and "Double" in _err()
    assert f(1, NULL, 8, 3, 3, 8, NULL, NULL) == INVALID and "null" in _err()
    assert f(1, NULL, -1, 3, 3, 8, NULL, NULL) == INVALID
    assert f(1, NULL, 0, 3, 3, 8, NULL, NULL) == 0                   # empty: nothing to do


def _msda(step=64, b=2, nq=4, force=0):
    return _bevk.lib().bevk_msda_forward(0, NULL, NULL, NULL, NULL, NULL, b, 10, 8, 32, 1, nq, 4,
                                         step, force, NULL, NULL)


def test_msda_validation():
    assert _msda(step=0) == INVALID and "im2col_step" in _err()
    assert _msda(b=6, step=4) == INVALID and "batch must divide im2col_step" in _err()
    assert _msda() == INVALID and "null" in _err()
    assert _msda(nq=0) == 0
    assert _msda(b=0) == 0


def _msda_bwd(dtype=0, step=64, b=2, nq=4, ws=0):
    return _bevk.lib().bevk_msda_backward(dtype, NULL, NULL, NULL, NULL, NULL, NULL,
                                          nq * 256, 256, 32, 1, b, 10, 8, 32, 1, nq, 4, step,
                                          0, NULL, NULL, NULL, NULL, ws, NULL)


def _sorted_bytes(b, s, h, nl, nq, np_):
    """Buffers of the sorted grad_value path: bucket counts, cursors and offsets (buckets of
    256 positions per (batch, head) slice), 8 per-XCD lists of 16-byte chunk headers (at
    most 3584 records each), and for every possible record (one per image row of a
    sample's corners: 2 per sample) an 8-byte weight pair and a 4-byte query / position
    word; each region 256-byte aligned."""
    up = lambda x: -(-x // 256) * 256  # noqa: E731
    nbs = -(-s // 256)
    cap = b * nq * h * nl * np_ * 2
    nbk = b * h * nbs
    items = -(-cap // 3584) + nbk
    return (2 * up(nbk * 4) + up((nbk + 1) * 4) + up(32) + up(8 * items * 16) + up(cap * 8)
            + up(cap * 4))


def test_msda_backward_workspace_bytes():
    f = _bevk.lib().bevk_msda_backward_workspace_bytes
    acc = lambda n: -(-n * 4 // 256) * 256  # noqa: E731
    # D != 32 and float64: only the 16-bit accumulator
    assert f(0, 2, 10, 8, 16, 1, 4, 4) == 0
    assert f(3, 2, 10, 8, 32, 1, 4, 4) == 0
    assert f(1, 2, 10, 8, 16, 1, 4, 4) == 2 * 10 * 8 * 16 * 4
    # D == 32: the sorted path's buffers (after the accumulator for 16-bit types)
    assert f(0, 2, 10, 8, 32, 1, 4, 4) == _sorted_bytes(2, 10, 8, 1, 4, 4)
    assert f(1, 2, 10, 8, 32, 1, 4, 4) == acc(2 * 10 * 8 * 32) + _sorted_bytes(2, 10, 8, 1, 4, 4)
    assert f(2, 6, 30825, 8, 32, 4, 10000, 8) == (acc(6 * 30825 * 8 * 32)
                                                 + _sorted_bytes(6, 30825, 8, 4, 10000, 8))
    assert f(4, 2, 10, 8, 32, 1, 4, 4) == -1
    assert f(1, -1, 10, 8, 32, 1, 4, 4) == -1
    assert f(1, 2, 10, 8, 32, 1, -4, 4) == -1


def test_msda_backward_validation():
    assert _msda_bwd(step=0) == INVALID and "im2col_step" in _err()
    assert _msda_bwd(b=6, step=4) == INVALID and "batch must divide im2col_step" in _err()
    assert _msda_bwd() == INVALID and "null" in _err()
    assert _msda_bwd(dtype=1) == INVALID and "workspace" in _err()
    assert _msda_bwd(dtype=1, ws=2 * 10 * 8 * 32 * 4) == INVALID and "null" in _err()
    assert _msda_bwd(dtype=7) == INVALID and "dtype" in _err()
    assert _msda_bwd(nq=0) == 0                     # f32: nothing to add
    assert _msda_bwd(b=0) == 0


def test_call_raises_runtime_error_with_message():
    with pytest.raises(RuntimeError, match="batch must divide im2col_step"):
        _bevk.call("bevk_msda_forward", 0, NULL, NULL, NULL, NULL, NULL, 6, 10, 8, 32, 1, 4, 4,
                   4, 0, NULL, NULL)


def test_col2im_nchw_rejects_misaligned_half_grad_im():
    """16-bit grad_im is added to with packed pair atomics, so it must start a 4-byte
    pair; a view at an odd element offset is rejected before any launch (fake device
    addresses: nothing is dereferenced)."""
    f = _bevk.lib().bevk_modulated_deformable_col2im_nchw
    p = ctypes.c_void_p
    args = [p(0x10000), p(0x20000), p(0x30000), p(0x40000), 1, 4, 5, 5, 5, 5, 3, 3, 1, 1, 1, 1,
            1, 1, 1]
    for dtype in (1, 2):
        assert f(dtype, *args, p(0x50002), NULL, NULL, NULL) == INVALID
        assert "aligned" in _err()


def _offset_conv(entry, dtype=1, **kw):
    a = dict(b=1, c=64, h=5, w=5, ho=5, wo=5, kh=3, kw=3, ph=1, pw=1, sh=1, sw=1, dh=1, dw=1)
    a.update(kw)
    sizes = [a[k] for k in ("b", "c", "h", "w", "ho", "wo")]
    geom = [a[k] for k in ("kh", "kw", "ph", "pw", "sh", "sw", "dh", "dw")]
    lib = _bevk.lib()
    if entry == "bevk_dcn_offset_conv_nhwc":
        return lib.bevk_dcn_offset_conv_nhwc(dtype, NULL, NULL, NULL, *sizes, *geom, NULL, NULL)
    return lib.bevk_dcn_mega_fwd_nhwc(dtype, NULL, NULL, NULL, NULL, NULL, *sizes,
                                      a.get("cout", 16), *geom, 0, NULL, NULL, NULL)


@pytest.mark.parametrize("entry", ["bevk_dcn_offset_conv_nhwc", "bevk_dcn_mega_fwd_nhwc"])
def test_offset_conv_validation(entry):
    assert _offset_conv(entry, dtype=3) == UNSUPPORTED and "not implemented" in _err()
    assert _offset_conv(entry, c=12) == UNSUPPORTED and "multiple of 8" in _err()
    assert _offset_conv(entry, kh=5, kw=5, ph=2, pw=2) == UNSUPPORTED and "9 taps" in _err()
    assert _offset_conv(entry, ho=4) == INVALID and "does not match" in _err()
    assert _offset_conv(entry) == INVALID and "null" in _err()
    assert _offset_conv(entry, b=0) == 0          # nothing to do


def test_noalloc_front_end_rejects_oversize_before_device_work():
    """The allocation-free front end checks its scratch need (here y alone: 160000 x 27 x
    4 bytes) against its 16 MiB static scratch before touching the device (fake
    addresses: nothing is dereferenced, no HIP call is made)."""
    f = _bevk.lib().bevk_modulated_deformable_fused_im2col_nhwc_noalloc
    p = ctypes.c_void_p
    rc = f(1, p(0x10000), p(0x20000), p(0x30000), 1, 16, 400, 400, 400, 400, 3, 3, 1, 1, 1, 1,
           1, 1, 1, p(0x40000), NULL)
    assert rc == INVALID and "static scratch" in _err()
