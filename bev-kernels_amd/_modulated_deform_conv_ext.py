"""The extension module of the reference, re-implemented over libbevk.so.

Same module name, function names and argument order as the reference's pybind11
module (naotic/bev-kernels csrc/binding.cpp:142-191), plus the MSDA ``forward`` /
``backward`` of its MUSA module (csrc_musa/msda/binding_musa.mu:545-557) and the fused
NHWC entry point ``dcn_fused_fwd_nhwc`` with its weight packer ``dcn_pack_weight``. Outputs are caller-allocated, as in the
reference (MSDA forward allocates and returns its output).

Unlike the reference launchers these wrappers check device, contiguity, dtype and
element counts against the integer sizes before launching, and raise RuntimeError on
a mismatch, so a kernel never indexes past a buffer.

The backward entry points (the col2im / col2im_coord names and MSDA ``backward``) run
the column-to-image and MSDA backward kernels of the library with the reference's
ownership rules: gradients the reference accumulates into caller-zeroed tensors are
added to what the caller passes, everything else is written.
"""
from __future__ import annotations

import os

import torch

import _bevk as _b

__all__ = [
    "modulated_deformable_im2col_cuda",
    "modulated_deformable_col2im_cuda",
    "modulated_deformable_im2col_opt_cuda",
    "modulated_deformable_col2im_opt_cuda",
    "modulated_deformable_col2im_smem_cuda",
    "modulated_deformable_col2im_coord_cuda",
    "modulated_deformable_col2im_coord_opt_cuda",
    "modulated_deformable_im2col_nhwc_cuda",
    "modulated_deformable_fused_im2col_nhwc_cuda",
    "modulated_deformable_col2im_nhwc_cuda",
    "modulated_deformable_col2im_coord_nhwc_cuda",
    "modulated_deformable_gradx_smem_nhwc_cuda",
    "modulated_deformable_gradx_gather_nhwc_cuda",
    "modulated_deformable_col2im_fused_smem_nhwc_cuda",
    "modulated_deformable_col2im_perelem_nhwc_cuda",
    "modulated_deformable_col2im_perelem_smem_nhwc_cuda",
    "dcn_packed_weight_numel",
    "dcn_pack_weight",
    "dcn_fused_fwd_nhwc",
    "dcn_offset_conv_nhwc",
    "dcn_mega_fwd_nhwc",
    "transpose",
    "nchw_to_nhwc",
    "nhwc_to_nchw",
    "forward",
    "backward",
]


def _im2col_nchw(entry, fn, data_im, data_offset, data_mask, batch_size, channels, height_im,
                 width_im, height_col, width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h,
                 stride_w, dilation_h, dilation_w, deformable_group, data_col):
    _b.require_device(fn, data_im, data_offset, data_mask, data_col)
    _b.require_contiguous(fn, data_im=data_im, data_offset=data_offset, data_mask=data_mask,
                          data_col=data_col)
    _b.require_dtype(fn, data_im, data_offset=data_offset, data_mask=data_mask,
                     data_col=data_col)
    if deformable_group <= 0:
        raise RuntimeError(f"{fn}: deformable_group must be positive")
    taps = kernel_h * kernel_w
    plane = height_col * width_col
    _b.require_numel(fn, "data_im", data_im, batch_size * channels * height_im * width_im)
    _b.require_numel(fn, "data_offset", data_offset,
                     batch_size * deformable_group * 2 * taps * plane)
    _b.require_numel(fn, "data_mask", data_mask, batch_size * deformable_group * taps * plane)
    _b.require_numel(fn, "data_col", data_col, channels * taps * batch_size * plane)
    _b.call(entry, _b.dtype_code(data_im), _b.ptr(data_im), _b.ptr(data_offset),
            _b.ptr(data_mask), batch_size, channels, height_im, width_im, height_col, width_col,
            kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
            deformable_group, _b.ptr(data_col), _b.stream_of(data_im))


def modulated_deformable_im2col_cuda(data_im, data_offset, data_mask, batch_size, channels,
                                     height_im, width_im, height_col, width_col, kernel_h,
                                     kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h,
                                     dilation_w, deformable_group, data_col):
    """NCHW modulated im2col into data_col [C*kh*kw, B, Ho, Wo] (binding.cpp:5-11)."""
    _im2col_nchw("bevk_modulated_deformable_im2col", "modulated_deformable_im2col_cuda",
                 data_im, data_offset, data_mask, batch_size, channels, height_im, width_im,
                 height_col, width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w,
                 dilation_h, dilation_w, deformable_group, data_col)


def modulated_deformable_im2col_opt_cuda(data_im, data_offset, data_mask, batch_size,
                                         channels, height_im, width_im, height_col, width_col,
                                         kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w,
                                         dilation_h, dilation_w, deformable_group, data_col):
    """Tiled NCHW modulated im2col, same contract (binding.cpp:21-27)."""
    _im2col_nchw("bevk_modulated_deformable_im2col_opt", "modulated_deformable_im2col_opt_cuda",
                 data_im, data_offset, data_mask, batch_size, channels, height_im, width_im,
                 height_col, width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w,
                 dilation_h, dilation_w, deformable_group, data_col)


def modulated_deformable_im2col_nhwc_cuda(data_im, data_offset, data_mask, batch_size,
                                          channels, height_im, width_im, height_col,
                                          width_col, kernel_h, kernel_w, pad_h, pad_w,
                                          stride_h, stride_w, dilation_h, dilation_w,
                                          deformable_group, data_col):
    """NHWC deformable gather into data_col [B*Ho*Wo, T*C] (binding.cpp:64-70).

    data_offset's last dim selects the form: 2T = offsets with a separate mask,
    3T = raw offset-conv output (offsets, then the pre-sigmoid mask)."""
    fn = "modulated_deformable_im2col_nhwc_cuda"
    if deformable_group != 1:
        raise RuntimeError("NHWC fused path supports deformable_group == 1 only")
    _b.require_device(fn, data_im, data_offset, data_mask, data_col)
    _b.require_contiguous(fn, data_im=data_im, data_offset=data_offset, data_mask=data_mask,
                          data_col=data_col)
    taps = kernel_h * kernel_w
    last = data_offset.size(-1)
    fused_y = last == 3 * taps
    _b.require_dtype(fn, data_im, data_offset=data_offset, data_col=data_col,
                     data_mask=None if fused_y else data_mask)
    m = batch_size * height_col * width_col
    _b.require_numel(fn, "data_im", data_im, batch_size * height_im * width_im * channels)
    _b.require_numel(fn, "data_offset", data_offset, m * last)
    if not fused_y:
        _b.require_numel(fn, "data_mask", data_mask, m * taps)
    _b.require_numel(fn, "data_col", data_col, m * taps * channels)
    _b.call("bevk_modulated_deformable_im2col_nhwc", _b.dtype_code(data_im), _b.ptr(data_im),
            _b.ptr(data_offset), last, _b.ptr(data_mask), batch_size, channels, height_im,
            width_im, height_col, width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h,
            stride_w, dilation_h, dilation_w, deformable_group, _b.ptr(data_col),
            _b.stream_of(data_im))


def dcn_packed_weight_numel(dtype, channels_out, kernel_h, kernel_w, channels):
    """Elements of the packed weight dcn_fused_fwd_nhwc takes for this shape and dtype."""
    code = _b._DTYPE_CODES.get(dtype)
    if code is None or code == _b.BEVK_F64:
        raise RuntimeError(f"dcn_pack_weight: dtype {dtype} is not supported")
    nbytes = _b.lib().bevk_dcn_packed_weight_bytes(code, channels_out, kernel_h, kernel_w,
                                                    channels)
    if nbytes < 0:
        raise RuntimeError("dcn_pack_weight: invalid weight shape")
    return nbytes // torch.empty((), dtype=dtype).element_size()


def dcn_pack_weight(weight, packed=None):
    """Module weight [Cout, C, kh, kw] -> the fused kernel's packed weight (1-D, same dtype).

    fp32: [Cout, kh, kw, C]; fp16 / bf16: MFMA-fragment blocks of 32 output channels x 16
    reduction elements (k = (i*kw + j)*C + c), zero padded. The reference permutes the
    weight to [kh, kw, C, Cout] on every call (fused_tl.py:500-510); the operator layer
    packs on every call as well (one small kernel)."""
    fn = "dcn_pack_weight"
    if weight.dim() != 4:
        raise RuntimeError(f"{fn}: weight must be [Cout, C, kh, kw], got {tuple(weight.shape)}")
    cout, c, kh, kw = weight.shape
    numel = dcn_packed_weight_numel(weight.dtype, cout, kh, kw, c)
    if packed is None:
        packed = weight.new_empty(numel)
    _b.require_device(fn, weight, packed)
    _b.require_contiguous(fn, weight=weight, packed=packed)
    _b.require_dtype(fn, weight, packed=packed)
    _b.require_numel(fn, "packed", packed, numel)
    _b.call("bevk_dcn_pack_weight", _b.dtype_code(weight), _b.ptr(weight), cout, kh, kw, c,
            _b.ptr(packed), _b.stream_of(weight))
    return packed


def transpose(src, dst, batch, rows, cols):
    """dst[b][c][r] = src[b][r][c] over a contiguous [batch, rows, cols] source (fp32, fp16,
    bf16; a bit-exact copy)."""
    fn = "transpose"
    _b.require_device(fn, src, dst)
    _b.require_contiguous(fn, src=src, dst=dst)
    _b.require_dtype(fn, src, dst=dst)
    _b.require_numel(fn, "src", src, batch * rows * cols)
    _b.require_numel(fn, "dst", dst, batch * rows * cols)
    _b.call("bevk_transpose", _b.dtype_code(src), _b.ptr(src), _b.ptr(dst), batch, rows, cols,
            _b.stream_of(src))
    return dst


def nchw_to_nhwc(x):
    """[B, C, H, W] (contiguous) -> a new contiguous [B, H, W, C] tensor."""
    b, c, h, w = x.shape
    out = x.new_empty(b, h, w, c)
    return transpose(x.contiguous(), out, b, c, h * w)


def nhwc_to_nchw(x):
    """[B, H, W, C] (contiguous) -> a new contiguous [B, C, H, W] tensor."""
    b, h, w, c = x.shape
    out = x.new_empty(b, c, h, w)
    return transpose(x.contiguous(), out, b, h * w, c)


def dcn_fused_fwd_nhwc(data_im, data_offset, data_mask, weight_packed, bias, batch_size,
                       channels, height_im, width_im, height_col, width_col, channels_out,
                       kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h,
                       dilation_w, out):
    """Fused NHWC DCNv2 forward into out [B, Ho, Wo, Cout] with no column buffer.

    weight_packed is dcn_pack_weight(weight) of the [Cout, C, kh, kw] weight in the input
    dtype; bias is [Cout] in the input dtype or None; data_offset follows the 2T / 3T rule
    of modulated_deformable_im2col_nhwc_cuda."""
    fn = "dcn_fused_fwd_nhwc"
    _b.require_device(fn, data_im, data_offset, data_mask, weight_packed, bias, out)
    _b.require_contiguous(fn, data_im=data_im, data_offset=data_offset, data_mask=data_mask,
                          weight_packed=weight_packed, bias=bias, out=out)
    taps = kernel_h * kernel_w
    last = data_offset.size(-1)
    fused_y = last == 3 * taps
    _b.require_dtype(fn, data_im, data_offset=data_offset, weight_packed=weight_packed,
                     bias=bias, out=out, data_mask=None if fused_y else data_mask)
    m = batch_size * height_col * width_col
    _b.require_numel(fn, "data_im", data_im, batch_size * height_im * width_im * channels)
    _b.require_numel(fn, "data_offset", data_offset, m * last)
    if not fused_y:
        _b.require_numel(fn, "data_mask", data_mask, m * taps)
    _b.require_numel(fn, "weight_packed", weight_packed,
                     dcn_packed_weight_numel(data_im.dtype, channels_out, kernel_h, kernel_w,
                                             channels))
    if bias is not None:
        _b.require_numel(fn, "bias", bias, channels_out)
    _b.require_numel(fn, "out", out, m * channels_out)
    _b.call("bevk_dcn_fused_fwd_nhwc", _b.dtype_code(data_im), _b.ptr(data_im),
            _b.ptr(data_offset), last, _b.ptr(data_mask), _b.ptr(weight_packed),
            _b.ptr(bias), batch_size, channels, height_im, width_im, height_col, width_col,
            channels_out, kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h,
            dilation_w, _b.ptr(out), _b.stream_of(data_im))


def _offset_conv_checks(fn, data_im, w_off_packed, b_off, batch_size, channels, height_im,
                        width_im, height_col, width_col, kernel_h, kernel_w, y):
    _b.require_contiguous(fn, data_im=data_im, w_off_packed=w_off_packed, b_off=b_off, y=y)
    _b.require_dtype(fn, data_im, w_off_packed=w_off_packed)
    for name, t in (("b_off", b_off), ("y", y)):
        if t is not None and t.dtype != torch.float32:
            raise RuntimeError(f"{fn}: {name} must be float32, got {t.dtype}")
    taps = kernel_h * kernel_w
    m = batch_size * height_col * width_col
    _b.require_numel(fn, "data_im", data_im, batch_size * height_im * width_im * channels)
    _b.require_numel(fn, "w_off_packed", w_off_packed,
                     dcn_packed_weight_numel(data_im.dtype, 3 * taps, kernel_h, kernel_w,
                                             channels))
    if b_off is not None:
        _b.require_numel(fn, "b_off", b_off, 3 * taps)
    _b.require_numel(fn, "y", y, m * 3 * taps)


def dcn_offset_conv_nhwc(data_im, w_off_packed, b_off, batch_size, channels, height_im,
                         width_im, height_col, width_col, kernel_h, kernel_w, pad_h, pad_w,
                         stride_h, stride_w, dilation_h, dilation_w, y):
    """Offset conv of the NHWC front end: y [B*Ho*Wo, 3T] (float32) = conv(x, w_off) +
    b_off with fp32 accumulation (the kernel of fused_tl.offset_conv_forward_nhwc,
    fused_tl.py:419-470). w_off_packed is dcn_pack_weight(w_off [3T, C, kh, kw]); b_off is
    float32 [3T] or None."""
    fn = "dcn_offset_conv_nhwc"
    _b.require_device(fn, data_im, w_off_packed, b_off, y)
    _offset_conv_checks(fn, data_im, w_off_packed, b_off, batch_size, channels, height_im,
                        width_im, height_col, width_col, kernel_h, kernel_w, y)
    _b.call("bevk_dcn_offset_conv_nhwc", _b.dtype_code(data_im), _b.ptr(data_im),
            _b.ptr(w_off_packed), _b.ptr(b_off), batch_size, channels, height_im, width_im,
            height_col, width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w,
            dilation_h, dilation_w, _b.ptr(y), _b.stream_of(data_im))


def dcn_mega_fwd_nhwc(data_im, w_off_packed, b_off, weight_packed, bias, batch_size, channels,
                      height_im, width_im, height_col, width_col, channels_out, kernel_h,
                      kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                      act_relu, y, out):
    """Whole DCNv2 forward with the offset conv inside (fused_tl.py:565-766 and the
    DCNSplitNHWCFunction forward with its ReLU epilogue, dcn_split_nhwc.py:158-204):
    y [B*Ho*Wo, 3T] float32 = conv(x, w_off) + b_off (written), offsets y[:, :2T], mask
    sigmoid(y[:, 2T:]), out [B, Ho, Wo, Cout] = deformable conv + bias (relu if act_relu).
    One kernel launch on the shapes of the persistent fp16/bf16 kernel."""
    fn = "dcn_mega_fwd_nhwc"
    _b.require_device(fn, data_im, w_off_packed, b_off, weight_packed, bias, y, out)
    _offset_conv_checks(fn, data_im, w_off_packed, b_off, batch_size, channels, height_im,
                        width_im, height_col, width_col, kernel_h, kernel_w, y)
    _b.require_contiguous(fn, weight_packed=weight_packed, bias=bias, out=out)
    _b.require_dtype(fn, data_im, weight_packed=weight_packed, bias=bias, out=out)
    m = batch_size * height_col * width_col
    _b.require_numel(fn, "weight_packed", weight_packed,
                     dcn_packed_weight_numel(data_im.dtype, channels_out, kernel_h, kernel_w,
                                             channels))
    if bias is not None:
        _b.require_numel(fn, "bias", bias, channels_out)
    _b.require_numel(fn, "out", out, m * channels_out)
    _b.call("bevk_dcn_mega_fwd_nhwc", _b.dtype_code(data_im), _b.ptr(data_im),
            _b.ptr(w_off_packed), _b.ptr(b_off), _b.ptr(weight_packed), _b.ptr(bias),
            batch_size, channels, height_im, width_im, height_col, width_col, channels_out,
            kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
            1 if act_relu else 0, _b.ptr(y), _b.ptr(out), _b.stream_of(data_im))


def _col2im_nchw(fn, data_col, data_im, data_offset, data_mask, batch_size, channels,
                 height_im, width_im, height_col, width_col, kernel_h, kernel_w, pad_h, pad_w,
                 stride_h, stride_w, dilation_h, dilation_w, deformable_group, grad_im,
                 grad_offset, grad_mask):
    _b.require_device(fn, data_col, data_im, data_offset, data_mask, grad_im, grad_offset,
                      grad_mask)
    _b.require_contiguous(fn, data_col=data_col, data_im=data_im, data_offset=data_offset,
                          data_mask=data_mask, grad_im=grad_im, grad_offset=grad_offset,
                          grad_mask=grad_mask)
    _b.require_dtype(fn, data_col, data_im=data_im, data_offset=data_offset,
                     data_mask=data_mask, grad_im=grad_im, grad_offset=grad_offset,
                     grad_mask=grad_mask)
    if deformable_group <= 0:
        raise RuntimeError(f"{fn}: deformable_group must be positive")
    taps = kernel_h * kernel_w
    plane = height_col * width_col
    _b.require_numel(fn, "data_col", data_col, channels * taps * batch_size * plane)
    if data_im is not None:
        _b.require_numel(fn, "data_im", data_im, batch_size * channels * height_im * width_im)
    _b.require_numel(fn, "data_offset", data_offset,
                     batch_size * deformable_group * 2 * taps * plane)
    _b.require_numel(fn, "data_mask", data_mask, batch_size * deformable_group * taps * plane)
    if grad_im is not None:
        _b.require_numel(fn, "grad_im", grad_im, batch_size * channels * height_im * width_im)
    if grad_offset is not None:
        _b.require_numel(fn, "grad_offset", grad_offset,
                         batch_size * deformable_group * 2 * taps * plane)
        _b.require_numel(fn, "grad_mask", grad_mask,
                         batch_size * deformable_group * taps * plane)
    _b.call("bevk_modulated_deformable_col2im_nchw", _b.dtype_code(data_col),
            _b.ptr(data_col), _b.ptr(data_im), _b.ptr(data_offset), _b.ptr(data_mask),
            batch_size, channels, height_im, width_im, height_col, width_col, kernel_h,
            kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
            deformable_group, _b.ptr(grad_im), _b.ptr(grad_offset), _b.ptr(grad_mask),
            _b.stream_of(data_col))


def _col2im_entry(name):
    def fn(data_col, data_offset, data_mask, batch_size, channels, height_im, width_im,
           height_col, width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w,
           dilation_h, dilation_w, deformable_group, grad_im):
        _col2im_nchw(name, data_col, None, data_offset, data_mask, batch_size, channels,
                     height_im, width_im, height_col, width_col, kernel_h, kernel_w, pad_h,
                     pad_w, stride_h, stride_w, dilation_h, dilation_w, deformable_group,
                     grad_im, None, None)
    fn.__name__ = name
    fn.__doc__ = ("NCHW backward column-to-image: grad_im [B,C,H,W] (input dtype) "
                  "accumulated from data_col [C*kh*kw, B*Ho*Wo]; zero it first.")
    return fn


def _col2im_coord_entry(name):
    def fn(data_col, data_im, data_offset, data_mask, batch_size, channels, height_im,
           width_im, height_col, width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h,
           stride_w, dilation_h, dilation_w, deformable_group, grad_offset, grad_mask):
        _col2im_nchw(name, data_col, data_im, data_offset, data_mask, batch_size, channels,
                     height_im, width_im, height_col, width_col, kernel_h, kernel_w, pad_h,
                     pad_w, stride_h, stride_w, dilation_h, dilation_w, deformable_group,
                     None, grad_offset, grad_mask)
    fn.__name__ = name
    fn.__doc__ = ("NCHW backward: grad_offset [B,dg*2T,Ho,Wo] and grad_mask [B,dg*T,Ho,Wo] "
                  "(input dtype), written.")
    return fn


# binding.cpp:13-19, :29-58. One kernel serves the reference's variants of each step.
modulated_deformable_col2im_cuda = _col2im_entry("modulated_deformable_col2im_cuda")
modulated_deformable_col2im_opt_cuda = _col2im_entry("modulated_deformable_col2im_opt_cuda")
modulated_deformable_col2im_smem_cuda = _col2im_entry("modulated_deformable_col2im_smem_cuda")
modulated_deformable_col2im_coord_cuda = _col2im_coord_entry(
    "modulated_deformable_col2im_coord_cuda")
modulated_deformable_col2im_coord_opt_cuda = _col2im_coord_entry(
    "modulated_deformable_col2im_coord_opt_cuda")


def _col2im_nhwc(fn, dcol, data_im, data_offset, data_mask, batch_size, channels, height_im,
                 width_im, height_col, width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h,
                 stride_w, dilation_h, dilation_w, deformable_group, grad_im, grad_offset,
                 grad_mask):
    if deformable_group != 1:
        raise RuntimeError("NHWC fused path supports deformable_group == 1 only")
    _b.require_device(fn, dcol, data_im, data_offset, data_mask, grad_im, grad_offset,
                      grad_mask)
    _b.require_contiguous(fn, dcol=dcol, data_im=data_im, data_offset=data_offset,
                          data_mask=data_mask, grad_im=grad_im, grad_offset=grad_offset,
                          grad_mask=grad_mask)
    taps = kernel_h * kernel_w
    last = data_offset.size(-1)
    fused_y = last == 3 * taps
    _b.require_dtype(fn, dcol, data_im=data_im, data_offset=data_offset,
                     data_mask=None if fused_y else data_mask)
    for name, t in (("grad_im", grad_im), ("grad_offset", grad_offset),
                    ("grad_mask", grad_mask)):
        if t is not None and t.dtype != torch.float32:
            raise RuntimeError(f"{fn}: {name} must be float32, got {t.dtype}")
    m = batch_size * height_col * width_col
    _b.require_numel(fn, "dcol", dcol, m * taps * channels)
    if data_im is not None:
        _b.require_numel(fn, "data_im", data_im, batch_size * height_im * width_im * channels)
    _b.require_numel(fn, "data_offset", data_offset, m * last)
    if not fused_y:
        _b.require_numel(fn, "data_mask", data_mask, m * taps)
    if grad_im is not None:
        _b.require_numel(fn, "grad_im", grad_im, batch_size * height_im * width_im * channels)
    if grad_offset is not None:
        _b.require_numel(fn, "grad_offset", grad_offset, m * 2 * taps)
        _b.require_numel(fn, "grad_mask", grad_mask, m * taps)
    _b.call("bevk_modulated_deformable_col2im_nhwc", _b.dtype_code(dcol), _b.ptr(dcol),
            _b.ptr(data_im), _b.ptr(data_offset), last, _b.ptr(data_mask), batch_size,
            channels, height_im, width_im, height_col, width_col, kernel_h, kernel_w, pad_h,
            pad_w, stride_h, stride_w, dilation_h, dilation_w, deformable_group,
            _b.ptr(grad_im), _b.ptr(grad_offset), _b.ptr(grad_mask), _b.stream_of(dcol))


def modulated_deformable_col2im_nhwc_cuda(dcol, data_im, data_offset, data_mask, batch_size,
                                          channels, height_im, width_im, height_col, width_col,
                                          kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w,
                                          dilation_h, dilation_w, deformable_group, grad_im,
                                          grad_offset, grad_mask):
    """NHWC backward column-to-image (binding.cpp:80-86): grad_im [B,H,W,C] fp32 accumulated
    (zero it first), grad_offset [M,2T] / grad_mask [M,T] fp32 written. data_offset may be
    the raw offset-conv output y [..., 3T]; grad_mask is then the pre-sigmoid gradient."""
    _col2im_nhwc("modulated_deformable_col2im_nhwc_cuda", dcol, data_im, data_offset,
                 data_mask, batch_size, channels, height_im, width_im, height_col, width_col,
                 kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                 deformable_group, grad_im, grad_offset, grad_mask)


def modulated_deformable_col2im_coord_nhwc_cuda(dcol, data_im, data_offset, data_mask,
                                                batch_size, channels, height_im, width_im,
                                                height_col, width_col, kernel_h, kernel_w,
                                                pad_h, pad_w, stride_h, stride_w, dilation_h,
                                                dilation_w, deformable_group, grad_offset,
                                                grad_mask):
    """grad_offset / grad_mask only (binding.cpp:88-95)."""
    _col2im_nhwc("modulated_deformable_col2im_coord_nhwc_cuda", dcol, data_im, data_offset,
                 data_mask, batch_size, channels, height_im, width_im, height_col, width_col,
                 kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                 deformable_group, None, grad_offset, grad_mask)


def modulated_deformable_gradx_smem_nhwc_cuda(dcol, data_offset, data_mask, batch_size,
                                              channels, height_im, width_im, height_col,
                                              width_col, kernel_h, kernel_w, pad_h, pad_w,
                                              stride_h, stride_w, dilation_h, dilation_w,
                                              deformable_group, grad_im):
    """grad_im only (binding.cpp:97-103), accumulated into grad_im."""
    _col2im_nhwc("modulated_deformable_gradx_smem_nhwc_cuda", dcol, None, data_offset,
                 data_mask, batch_size, channels, height_im, width_im, height_col, width_col,
                 kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                 deformable_group, grad_im, None, None)


def modulated_deformable_gradx_gather_nhwc_cuda(dcol, data_offset, data_mask, batch_size,
                                                channels, height_im, width_im, height_col,
                                                width_col, kernel_h, kernel_w, pad_h, pad_w,
                                                stride_h, stride_w, dilation_h, dilation_w,
                                                deformable_group, win, grad_im):
    """grad_im only (binding.cpp:105-111). `win` (the reference's gather search window) has
    no meaning here: every sample scatters its own corners."""
    _col2im_nhwc("modulated_deformable_gradx_gather_nhwc_cuda", dcol, None, data_offset,
                 data_mask, batch_size, channels, height_im, width_im, height_col, width_col,
                 kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                 deformable_group, grad_im, None, None)


modulated_deformable_col2im_fused_smem_nhwc_cuda = modulated_deformable_col2im_nhwc_cuda
modulated_deformable_col2im_perelem_nhwc_cuda = modulated_deformable_col2im_nhwc_cuda
modulated_deformable_col2im_perelem_smem_nhwc_cuda = modulated_deformable_col2im_nhwc_cuda


def modulated_deformable_fused_im2col_nhwc_cuda(data_im, w_off, b_off, batch_size, channels,
                                                height_im, width_im, height_col, width_col,
                                                kernel_h, kernel_w, pad_h, pad_w, stride_h,
                                                stride_w, dilation_h, dilation_w,
                                                deformable_group, data_col):
    """Offset conv + sigmoid + NHWC gather (binding.cpp:72-78, dcn_fused_nhwc_cuda.cu:92-126).

    data_im [B, H, W, C]; w_off [3T, T, C] (the offset conv weight permuted (0, 2, 3, 1)) in
    the input dtype; b_off [3T] float32; data_col [B*Ho*Wo, T*C]. The offset conv runs on
    the matrix cores with fp32 accumulation and its output stays fp32."""
    fn = "modulated_deformable_fused_im2col_nhwc_cuda"
    if deformable_group != 1:
        raise RuntimeError("NHWC fused path supports deformable_group == 1 only")
    _b.require_device(fn, data_im, w_off, b_off, data_col)
    _b.require_contiguous(fn, data_im=data_im, w_off=w_off, b_off=b_off, data_col=data_col)
    _b.require_dtype(fn, data_im, w_off=w_off, data_col=data_col)
    if b_off.dtype != torch.float32:
        raise RuntimeError(f"{fn}: b_off must be float32, got {b_off.dtype}")
    taps = kernel_h * kernel_w
    m = batch_size * height_col * width_col
    _b.require_numel(fn, "data_im", data_im, batch_size * height_im * width_im * channels)
    _b.require_numel(fn, "w_off", w_off, 3 * taps * taps * channels)
    _b.require_numel(fn, "b_off", b_off, 3 * taps)
    _b.require_numel(fn, "data_col", data_col, m * taps * channels)
    code = _b.dtype_code(data_im)
    nbytes = _b.lib().bevk_dcn_fused_im2col_nhwc_workspace_bytes(
        code, batch_size, channels, height_col, width_col, kernel_h, kernel_w)
    if nbytes < 0:
        raise RuntimeError(f"{fn}: dtype {data_im.dtype} is not supported")
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=data_im.device)
    _b.call("bevk_modulated_deformable_fused_im2col_nhwc", code, _b.ptr(data_im), _b.ptr(w_off),
            _b.ptr(b_off), batch_size, channels, height_im, width_im, height_col, width_col,
            kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
            deformable_group, _b.ptr(ws), nbytes, _b.ptr(data_col), _b.stream_of(data_im))


# ---------------------------------------------------------------------------------------
# Multi-scale deformable attention (binding_musa.mu:286-412, :545-557)
# ---------------------------------------------------------------------------------------

def _msda_check(fn, value, spatial_shapes, level_start_index, sampling_loc, attn_weight):
    """Checks of binding_musa.mu:292-298 / :420-427 plus shape agreement; returns
    (batch, spatial, heads, channels, num_levels, num_query, num_point)."""
    if value.device.type != "cuda":
        raise RuntimeError("value must be a HIP device tensor")
    if not value.is_contiguous():
        raise RuntimeError("value must be contiguous")
    if not spatial_shapes.is_contiguous():
        raise RuntimeError("spatial_shapes must be contiguous")
    if not level_start_index.is_contiguous():
        raise RuntimeError("level_start_index must be contiguous")
    if not sampling_loc.is_contiguous():
        raise RuntimeError("sampling_loc must be contiguous")
    if not attn_weight.is_contiguous():
        raise RuntimeError("attn_weight must be contiguous")
    _b.require_device(fn, value, spatial_shapes, level_start_index, sampling_loc, attn_weight)
    _b.require_dtype(fn, value, sampling_loc=sampling_loc, attn_weight=attn_weight)
    if spatial_shapes.dtype != torch.int64 or level_start_index.dtype != torch.int64:
        raise RuntimeError(f"{fn}: spatial_shapes and level_start_index must be int64")
    if value.dim() != 4 or sampling_loc.dim() != 6 or attn_weight.dim() != 5:
        raise RuntimeError(
            f"{fn}: expected value [B,S,heads,D], sampling_loc [B,Lq,heads,L,P,2] and "
            "attn_weight [B,Lq,heads,L,P]")
    batch, spatial, heads, channels = value.shape
    num_levels = spatial_shapes.size(0)
    num_query = sampling_loc.size(1)
    num_point = sampling_loc.size(4)
    if tuple(spatial_shapes.shape) != (num_levels, 2) or \
            tuple(level_start_index.shape) != (num_levels,):
        raise RuntimeError(f"{fn}: spatial_shapes must be [L, 2] and level_start_index [L]")
    if tuple(sampling_loc.shape) != (batch, num_query, heads, num_levels, num_point, 2):
        raise RuntimeError(f"{fn}: sampling_loc shape {tuple(sampling_loc.shape)} does not match "
                           f"value {tuple(value.shape)} and {num_levels} levels")
    if tuple(attn_weight.shape) != (batch, num_query, heads, num_levels, num_point):
        raise RuntimeError(f"{fn}: attn_weight shape {tuple(attn_weight.shape)} does not match "
                           f"sampling_loc {tuple(sampling_loc.shape)}")
    return batch, spatial, heads, channels, num_levels, num_query, num_point


def forward(value, spatial_shapes, level_start_index, sampling_loc, attn_weight,
            im2col_step=64, force_generic=False):
    """MSDA forward. value [B, S, heads, D], spatial_shapes [L, 2] int64,
    level_start_index [L] int64, sampling_loc [B, Lq, heads, L, P, 2],
    attn_weight [B, Lq, heads, L, P] -> output [B, Lq, heads * D]."""
    batch, spatial, heads, channels, num_levels, num_query, num_point = _msda_check(
        "msda_forward", value, spatial_shapes, level_start_index, sampling_loc, attn_weight)
    output = torch.empty(batch, num_query, heads * channels, dtype=value.dtype,
                         device=value.device)
    _b.call("bevk_msda_forward", _b.dtype_code(value), _b.ptr(value), _b.ptr(spatial_shapes),
            _b.ptr(level_start_index), _b.ptr(sampling_loc), _b.ptr(attn_weight), batch, spatial,
            heads, channels, num_levels, num_query, num_point, int(im2col_step),
            1 if force_generic else 0, _b.ptr(output), _b.stream_of(value))
    return output


MSDA_BACKWARD_MAX_WORKSPACE_ENV = "BEVK_MSDA_BACKWARD_MAX_WORKSPACE"


def _workspace_cap(max_workspace_bytes):
    """The byte cap on the backward's scratch: the argument, else the environment variable
    BEVK_MSDA_BACKWARD_MAX_WORKSPACE (bytes), else none."""
    if max_workspace_bytes is not None:
        return int(max_workspace_bytes)
    env = os.environ.get(MSDA_BACKWARD_MAX_WORKSPACE_ENV)
    if env is None or env.strip() == "":
        return None
    try:
        return int(env)
    except ValueError:
        raise RuntimeError(f"{MSDA_BACKWARD_MAX_WORKSPACE_ENV}={env!r} is not a byte count")


def backward_workspace_bytes(value, num_levels, num_query, num_point, max_workspace_bytes=None):
    """(bytes the backward will ask for, the least it can run with) for value
    [B, S, heads, D]: bevk_msda_backward_workspace_bytes, or the least when that is above
    the cap (_workspace_cap). The least is the fp32 grad_value accumulator of 16-bit types
    and nothing for fp32 / fp64."""
    batch, spatial, heads, channels = value.shape
    full = _b.lib().bevk_msda_backward_workspace_bytes(_b.dtype_code(value), batch, spatial,
                                                        heads, channels, num_levels, num_query,
                                                        num_point)
    if full < 0:
        raise RuntimeError("msda_backward: invalid sizes")
    least = value.numel() * 4 if value.dtype in (torch.float16, torch.bfloat16) else 0
    cap = _workspace_cap(max_workspace_bytes)
    if cap is not None and full > max(cap, least):
        return least, least
    return full, least


def backward(value, spatial_shapes, level_start_index, sampling_loc, attn_weight, grad_output,
             grad_value, grad_sampling_loc, grad_attn_weight, im2col_step=64,
             force_generic_col2im=False, max_workspace_bytes=None):
    """MSDA backward (binding_musa.mu:414-543). Fills the caller's tensors:
    grad_value [B, S, heads, D] is ADDED to for fp32/fp64 and overwritten for fp16/bf16
    (accumulated in an fp32 buffer, then narrowed); grad_sampling_loc and
    grad_attn_weight are written. grad_output [B, Lq, heads*D] may be strided.

    Scratch: with head_dim 32 the fastest kernels (grad_value by a bucket sort of the
    samples, no per-corner atomics) take bevk_msda_backward_workspace_bytes of device
    memory, about 12 bytes per (sample, corner row) on top of the fp32 accumulator 16-bit
    types need (SCA, 6 cameras: 370 MB fp32, 560 MB fp16). When that exceeds
    max_workspace_bytes (default: the BEVK_MSDA_BACKWARD_MAX_WORKSPACE environment
    variable; unset = no cap), or its allocation fails, the call passes only the least
    workspace and the library runs the atomic kernels instead, as the reference does: no
    scratch for fp32 / fp64, the fp32 grad_value accumulator for fp16 / bf16
    (binding_musa.mu:456-467). The accumulator is needed whatever the cap."""
    fn = "msda_backward"
    batch, spatial, heads, channels, num_levels, num_query, num_point = _msda_check(
        fn, value, spatial_shapes, level_start_index, sampling_loc, attn_weight)
    if grad_output.device.type != "cuda":
        raise RuntimeError("grad_output must be a HIP device tensor")
    _b.require_device(fn, value, grad_output, grad_value, grad_sampling_loc, grad_attn_weight)
    _b.require_dtype(fn, value, grad_output=grad_output, grad_value=grad_value,
                     grad_sampling_loc=grad_sampling_loc, grad_attn_weight=grad_attn_weight)
    _b.require_contiguous(fn, grad_value=grad_value, grad_sampling_loc=grad_sampling_loc,
                          grad_attn_weight=grad_attn_weight)
    if tuple(grad_value.shape) != tuple(value.shape) or \
            tuple(grad_sampling_loc.shape) != tuple(sampling_loc.shape) or \
            tuple(grad_attn_weight.shape) != tuple(attn_weight.shape):
        raise RuntimeError(f"{fn}: gradient tensors must have the shapes of value, "
                           "sampling_loc and attn_weight")
    # binding_musa.mu:446-447 views grad_output per (batch, query, head, channel)
    g4 = grad_output.view(batch, num_query, heads, channels)
    sb, sq, sh, sc = g4.stride()
    code = _b.dtype_code(value)
    nbytes, least = backward_workspace_bytes(value, num_levels, num_query, num_point,
                                             max_workspace_bytes)
    try:
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=value.device)
    except torch.OutOfMemoryError:
        if nbytes <= least:
            raise
        nbytes = least
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=value.device)
    _b.call("bevk_msda_backward", code, _b.ptr(value), _b.ptr(spatial_shapes),
            _b.ptr(level_start_index), _b.ptr(sampling_loc), _b.ptr(attn_weight), _b.ptr(g4),
            sb, sq, sh, sc, batch, spatial, heads, channels, num_levels, num_query, num_point,
            int(im2col_step), 1 if force_generic_col2im else 0, _b.ptr(grad_value),
            _b.ptr(grad_sampling_loc), _b.ptr(grad_attn_weight), _b.ptr(ws), nbytes,
            _b.stream_of(value))
