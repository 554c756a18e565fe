"""ctypes binding of libbevk.so (the gfx950 kernels) for the Python operator layer.

The library is loaded after torch so that it binds to the HIP runtime torch already
mapped: torch's streams and allocations are only valid in that runtime. A second
runtime in the process is treated as a fatal configuration error.

Every call goes through :func:`call`, which raises ``RuntimeError`` with the library's
message when an entry point returns a nonzero status.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be imported before the library is loaded)

_LIB_NAME = "libbevk.so"
_HERE = os.path.dirname(os.path.abspath(__file__))

BEVK_F32, BEVK_F16, BEVK_BF16, BEVK_F64 = 0, 1, 2, 3
_DTYPE_CODES = {
    torch.float32: BEVK_F32,
    torch.float16: BEVK_F16,
    torch.bfloat16: BEVK_BF16,
    torch.float64: BEVK_F64,
}

_vp = ctypes.c_void_p
_i = ctypes.c_int

# name -> argument types (after the leading dtype code where present)
_SIGNATURES = {
    "bevk_modulated_deformable_im2col": [_i, _vp, _vp, _vp] + [_i] * 15 + [_vp, _vp],
    "bevk_modulated_deformable_im2col_opt": [_i, _vp, _vp, _vp] + [_i] * 15 + [_vp, _vp],
    "bevk_modulated_deformable_im2col_nhwc": [_i, _vp, _vp, _i, _vp] + [_i] * 15 + [_vp, _vp],
    "bevk_modulated_deformable_col2im_nchw": [_i, _vp, _vp, _vp, _vp] + [_i] * 15
    + [_vp, _vp, _vp, _vp],
    "bevk_modulated_deformable_col2im_nhwc": [_i, _vp, _vp, _vp, _i, _vp] + [_i] * 15
    + [_vp, _vp, _vp, _vp],
    "bevk_dcn_fused_im2col_nhwc_workspace_bytes": [_i] * 7,
    "bevk_modulated_deformable_fused_im2col_nhwc": [_i, _vp, _vp, _vp] + [_i] * 15
    + [_vp, ctypes.c_int64, _vp, _vp],
    "bevk_modulated_deformable_fused_im2col_nhwc_noalloc": [_i, _vp, _vp, _vp] + [_i] * 15
    + [_vp, _vp],
    "bevk_dcn_packed_weight_bytes": [_i] * 5,
    "bevk_dcn_pack_weight": [_i, _vp] + [_i] * 4 + [_vp, _vp],
    "bevk_dcn_fused_fwd_nhwc": [_i, _vp, _vp, _i, _vp, _vp, _vp] + [_i] * 15 + [_vp, _vp],
    "bevk_transpose": [_i, _vp, _vp, _i, _i, _i, _vp],
    "bevk_dcn_offset_conv_nhwc": [_i, _vp, _vp, _vp] + [_i] * 14 + [_vp, _vp],
    "bevk_dcn_mega_fwd_nhwc": [_i, _vp, _vp, _vp, _vp, _vp] + [_i] * 16 + [_vp, _vp, _vp],
    "bevk_msda_forward": [_i, _vp, _vp, _vp, _vp, _vp] + [_i] * 9 + [_vp, _vp],
    "bevk_msda_backward_workspace_bytes": [_i] * 8,
    "bevk_msda_backward": [_i, _vp, _vp, _vp, _vp, _vp, _vp] + [ctypes.c_int64] * 4
    + [_i] * 9 + [_vp, _vp, _vp, _vp, ctypes.c_int64, _vp],
}

# entry points that return a value instead of a bevk_status
_RESTYPES = {"bevk_dcn_packed_weight_bytes": ctypes.c_int64,
             "bevk_dcn_fused_im2col_nhwc_workspace_bytes": ctypes.c_int64,
             "bevk_msda_backward_workspace_bytes": ctypes.c_int64}

_lib = None
_lock = threading.Lock()


def library_path() -> str:
    return os.environ.get("BEVK_LIBRARY", os.path.join(_HERE, _LIB_NAME))


def _hip_runtimes() -> set[str]:
    try:
        with open("/proc/self/maps") as f:
            return {line.split()[-1] for line in f if "libamdhip64" in line}
    except OSError:
        return set()


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is missing or mis-linked."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise ImportError(
                f"{path} not found: build the HIP kernels first "
                "(python setup.py build_ext --inplace)")
        handle = ctypes.CDLL(path)
        runtimes = _hip_runtimes()
        if len(runtimes) > 1:
            raise ImportError(
                "libbevk.so bound a second HIP runtime next to torch's: "
                + ", ".join(sorted(runtimes)))
        handle.bevk_last_error.restype = ctypes.c_char_p
        handle.bevk_last_error.argtypes = []
        handle.bevk_version.restype = ctypes.c_char_p
        handle.bevk_version.argtypes = []
        for name, args in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
            fn.argtypes = args
        _lib = handle
        return _lib


def exported_symbols() -> list[str]:
    return ["bevk_last_error", "bevk_version", *_SIGNATURES.keys()]


def version() -> str:
    return lib().bevk_version().decode()


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().bevk_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"{name} failed with status {rc}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODES[t.dtype]
    except KeyError:
        raise RuntimeError(f"dtype {t.dtype} is not supported by the bev-kernels library")


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    """Raw hipStream_t of torch's current stream on the tensor's device."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_device(fn: str, *tensors: torch.Tensor) -> torch.device:
    """All tensors on one HIP device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"{fn}: expected tensors on a HIP (cuda) device, got {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{fn}: tensors are on different devices ({dev}, {t.device})")
    return dev


def require_contiguous(fn: str, **tensors: torch.Tensor) -> None:
    for name, t in tensors.items():
        if t is not None and not t.is_contiguous():
            raise RuntimeError(f"{name} must be contiguous")


def require_numel(fn: str, name: str, t: torch.Tensor, expected: int) -> None:
    if t.numel() != expected:
        raise RuntimeError(
            f"{fn}: {name} has {t.numel()} elements, the given sizes need {expected}")


def require_dtype(fn: str, ref: torch.Tensor, **tensors: torch.Tensor) -> None:
    for name, t in tensors.items():
        if t is not None and t.dtype != ref.dtype:
            raise RuntimeError(f"{fn}: {name} has dtype {t.dtype}, expected {ref.dtype}")
