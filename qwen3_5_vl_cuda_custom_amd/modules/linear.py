"""CudaLinear (reference modules/linear.py:11-39)."""
from __future__ import annotations

import math

import torch
from torch import nn

from ..kernels import matmul


class CudaLinear(nn.Module):
    """Drop-in nn.Linear on the gfx950 MFMA GEMM; `weight` (out, in), `bias` (out) or None."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight = nn.Parameter(torch.empty(out_features, in_features))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            fan_in = self.weight.shape[1]
            bound = 1.0 / math.sqrt(fan_in) if fan_in > 0 else 0.0
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        """x·Wᵀ + b (+ residual, added in the GEMM epilogue before the single rounding)."""
        return matmul(x, self.weight, self.bias, residual=residual)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}"
