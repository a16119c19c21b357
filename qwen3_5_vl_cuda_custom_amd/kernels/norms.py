"""Row reductions: rmsnorm, layernorm, softmax (reference kernels/rmsnorm.py:66-77,
kernels/layernorm.py:54-68, kernels/softmax.py:40-51)."""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check
from .backward import LayerNormFunction, RMSNormFunction, SoftmaxFunction, needs_grad


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x·rsqrt(mean(x²)+eps)·w over the last dim, fp32 inside, rounded once."""
    if needs_grad(x, weight):
        return RMSNormFunction.apply(x, weight, eps)
    check("rmsnorm", x, weight)
    cols = x.shape[-1]
    if weight.shape != (cols,):
        raise ValueError(f"rmsnorm: weight {tuple(weight.shape)} != ({cols},)")
    x = x.contiguous()
    y = torch.empty_like(x)
    _lib.call("q3_rmsnorm", x.data_ptr(), weight.contiguous().data_ptr(), y.data_ptr(), x.numel() // cols, cols,
              float(eps), _lib.dtype_code(x.dtype), _lib.stream())
    return y


def layernorm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
              eps: float = 1e-6) -> torch.Tensor:
    """(x−μ)·rsqrt(var+eps)·w + b over the last dim (two-pass statistics in registers)."""
    if needs_grad(x, weight, bias):
        return LayerNormFunction.apply(x, weight, bias, eps)
    check("layernorm", x, weight, bias)
    cols = x.shape[-1]
    if weight.shape != (cols,) or (bias is not None and bias.shape != (cols,)):
        raise ValueError("layernorm: weight/bias must be (cols,)")
    x = x.contiguous()
    y = torch.empty_like(x)
    b = bias.contiguous() if bias is not None else None
    _lib.call("q3_layernorm", x.data_ptr(), weight.contiguous().data_ptr(), _lib.ptr(b), y.data_ptr(),
              x.numel() // cols, cols, float(eps), _lib.dtype_code(x.dtype), _lib.stream())
    return y


def softmax(x: torch.Tensor) -> torch.Tensor:
    """Row softmax over the last dim."""
    if needs_grad(x):
        return SoftmaxFunction.apply(x)
    check("softmax", x)
    cols = x.shape[-1]
    x = x.contiguous()
    y = torch.empty_like(x)
    _lib.call("q3_softmax", x.data_ptr(), y.data_ptr(), x.numel() // cols, cols, _lib.dtype_code(x.dtype),
              _lib.stream())
    return y
