"""Elementwise ops: residual_add, swiglu, gelu_tanh, sigmoid_mul (reference kernels/residual_add.py:28-39,
kernels/swiglu.py:56-67, kernels/gelu_tanh.py:49-60, kernels/sigmoid_mul.py:49-60); each differentiable."""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check
from .backward import (GeluTanhFunction, ResidualAddFunction, SigmoidMulFunction, SwiGLUFunction,
                       needs_grad)


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
    if needs_grad(a, b):
        return ResidualAddFunction.apply(a, b)
    return _binary("residual_add", a, b)


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate)·up in fp32, rounded once."""
    if needs_grad(gate, up):
        return SwiGLUFunction.apply(gate, up)
    return _binary("swiglu", gate, up)


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """0.5x(1+tanh(√(2/π)(x+0.044715x³)))."""
    if needs_grad(x):
        return GeluTanhFunction.apply(x)
    check("gelu_tanh", x)
    x = x.contiguous()
    y = torch.empty_like(x)
    _lib.call("q3_gelu_tanh", x.data_ptr(), y.data_ptr(), x.numel(), _lib.dtype_code(x.dtype), _lib.stream())
    return y


def sigmoid_mul(x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """x·sigmoid(gate) in fp32, rounded once (reference kernels/sigmoid_mul.py:49-60,
    csrc/sigmoid_mul_op.cu:5-16)."""
    if needs_grad(x, gate):
        return SigmoidMulFunction.apply(x, gate)
    return _binary("sigmoid_mul", x, gate)
