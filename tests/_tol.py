"""Parity tolerances (1e-4 abs/rel in fp32, 1e-2 rel in fp16/bf16
with fp32 accumulation):
  fp32:      |a - r| <= 1e-4 + 1e-4 * |r|                     elementwise
  fp16/bf16: |a - r| <= 1e-2 * |r| + 1e-2 * mean|r|           elementwise, i.e.
             allclose(rtol=1e-2, atol=1e-2 * mean|r|) (the norm SURVEY appendix A.3
             states; a pure elementwise relative error is undefined where r ~ 0)
The reference r is the float64 oracle evaluated on exactly the values the kernel saw
(inputs already rounded to the kernel's dtype). For bf16 the output rounding alone is up
to 2^-8 = 0.39% of |r|, and the deformable taps are rounded to bf16 before the matrix
cores, as in the reference's column buffer."""
from __future__ import annotations

import torch


def check_fp32(actual: torch.Tensor, ref: torch.Tensor, what: str = "") -> None:
    a = actual.detach().double().cpu()
    r = ref.detach().double().cpu()
    assert a.shape == r.shape, f"{what}: shape {tuple(a.shape)} != {tuple(r.shape)}"
    err = (a - r).abs()
    bound = 1e-4 + 1e-4 * r.abs()
    bad = ~(err <= bound)
    if bad.any():
        i = int(bad.flatten().nonzero()[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{a.numel()} elements outside 1e-4 abs+rel; max err "
            f"{err.max().item():.3e}; first bad flat index {i}: got {a.flatten()[i].item():.7g}"
            f" want {r.flatten()[i].item():.7g}")


def check_half(actual: torch.Tensor, ref: torch.Tensor, what: str = "") -> None:
    a = actual.detach().double().cpu()
    r = ref.detach().double().cpu()
    assert a.shape == r.shape, f"{what}: shape {tuple(a.shape)} != {tuple(r.shape)}"
    err = (a - r).abs()
    scale = r.abs() + r.abs().mean()
    bad = ~(err <= 1e-2 * scale)
    if bad.any():
        i = int(bad.flatten().nonzero()[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{a.numel()} elements outside 1e-2*(|r|+mean|r|); "
            f"max rel {(err / scale).max().item():.3e}; first bad flat index {i}: got "
            f"{a.flatten()[i].item():.7g} want {r.flatten()[i].item():.7g}")


def check(actual: torch.Tensor, ref: torch.Tensor, dtype: torch.dtype, what: str = "") -> None:
    if dtype in (torch.float16, torch.bfloat16):
        check_half(actual, ref, what)
    else:
        check_fp32(actual, ref, what)
