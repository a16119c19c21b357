"""Elementwise ops: residual_add, swiglu, gelu_tanh (reference kernels/residual_add.py:28-39,
kernels/swiglu.py:56-67, kernels/gelu_tanh.py:49-60)."""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check


def _binary(name: str, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    check(name, a, b)
    if a.shape != b.shape:
        raise ValueError(f"{name}: shapes differ {tuple(a.shape)} vs {tuple(b.shape)}")
    a, b = a.contiguous(), b.contiguous()
    y = torch.empty_like(a)
    _lib.call(f"q3_{name}", a.data_ptr(), b.data_ptr(), y.data_ptr(), a.numel(), _lib.dtype_code(a.dtype),
              _lib.stream())
    return y


def residual_add(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a + b (one rounding)."""
    return _binary("residual_add", a, b)


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate)·up in fp32, rounded once."""
    return _binary("swiglu", gate, up)


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """0.5x(1+tanh(√(2/π)(x+0.044715x³)))."""
    check("gelu_tanh", x)
    x = x.contiguous()
    y = torch.empty_like(x)
    _lib.call("q3_gelu_tanh", x.data_ptr(), y.data_ptr(), x.numel(), _lib.dtype_code(x.dtype), _lib.stream())
    return y
