"""CudaRMSNorm / CudaLayerNorm (reference modules/norms.py:9-42)."""
from __future__ import annotations

import torch
from torch import nn

from ..kernels import RMSNORM_MATMUL_MAX_ROWS, layernorm, rmsnorm


class CudaRMSNorm(nn.Module):
    """y = x·rsqrt(mean(x²)+eps)·weight; `weight` (dim) initialised to ones."""

    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.dim = dim
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rmsnorm(x, self.weight, self.eps)

    def extra_repr(self) -> str:
        return f"{self.dim}, eps={self.eps}"


def fused_norm_ok(x: torch.Tensor, norm: CudaRMSNorm) -> bool:
    """Whether `norm` can run inside the projection that consumes x
    (rmsnorm_matmul_segments / rmsnorm_matmul_swiglu): decode shapes of at most
    32 bf16 rows, 16-byte aligned rows of a multiple of 8 elements."""
    K = x.shape[-1]
    return (x.is_cuda and x.dtype == torch.bfloat16 and norm.weight.dtype == torch.bfloat16 and K == norm.dim
            and K % 8 == 0 and x.is_contiguous() and x.data_ptr() % 16 == 0
            and 0 < x.numel() // K <= RMSNORM_MATMUL_MAX_ROWS)


class CudaLayerNorm(nn.Module):
    """nn.LayerNorm parameter layout: `weight` ones, `bias` zeros (or None)."""

    def __init__(self, dim: int, eps: float = 1e-6, bias: bool = True) -> None:
        super().__init__()
        self.normalized_shape = (dim,)
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))
        if bias:
            self.bias = nn.Parameter(torch.zeros(dim))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return layernorm(x, self.weight, self.bias, self.eps)

    def extra_repr(self) -> str:
        return f"{self.normalized_shape[0]}, eps={self.eps}, bias={self.bias is not None}"
