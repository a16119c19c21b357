"""CudaSwiGLUMLP / CudaVisionMLP (reference modules/mlp.py:10-34)."""
from __future__ import annotations

import torch
from torch import nn

from ..kernels import gelu_tanh, matmul_gelu, matmul_swiglu, rmsnorm_matmul_swiglu, swiglu
from ..kernels.backward import needs_grad
from .linear import CudaLinear
from .norms import CudaRMSNorm, fused_norm_ok


class CudaSwiGLUMLP(nn.Module):
    """down_proj(silu(gate_proj(x)) · up_proj(x)); gate/up (I, h), down (h, I)."""

    def __init__(self, hidden_size: int, intermediate_size: int, bias: bool = False) -> None:
        super().__init__()
        self.gate_proj = CudaLinear(hidden_size, intermediate_size, bias=bias)
        self.up_proj = CudaLinear(hidden_size, intermediate_size, bias=bias)
        self.down_proj = CudaLinear(intermediate_size, hidden_size, bias=bias)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None, *,
                input_norm: CudaRMSNorm | None = None) -> torch.Tensor:
        """`input_norm`: x is taken before this RMSNorm; for decode shapes (at
        most 32 bf16 tokens) it runs inside the gate/up GEMM, else first."""
        if needs_grad(x, residual, *self.parameters()):  # training: modules/mlp.py:19-22 on differentiable ops
            if input_norm is not None:
                x = input_norm(x)
            return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x)), residual=residual)
        no_bias = self.gate_proj.bias is None and self.up_proj.bias is None
        if input_norm is not None and no_bias and fused_norm_ok(x, input_norm):
            act = rmsnorm_matmul_swiglu(x, input_norm.weight, input_norm.eps, self.gate_proj.weight,
                                        self.up_proj.weight)
            return self.down_proj(act, residual=residual)
        if input_norm is not None:
            x = input_norm(x)
        if no_bias:
            act = matmul_swiglu(x, self.gate_proj.weight, self.up_proj.weight)  # gate, up and swiglu in one GEMM
        else:
            act = swiglu(self.gate_proj(x), self.up_proj(x))
        return self.down_proj(act, residual=residual)


class CudaVisionMLP(nn.Module):
    """linear_fc2(gelu_tanh(linear_fc1(x))), both with bias; the gelu runs in fc1's GEMM epilogue."""

    def __init__(self, hidden_size: int, intermediate_size: int) -> None:
        super().__init__()
        self.linear_fc1 = CudaLinear(hidden_size, intermediate_size, bias=True)
        self.linear_fc2 = CudaLinear(intermediate_size, hidden_size, bias=True)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        if needs_grad(x, residual, *self.parameters()):  # training: modules/mlp.py:33-34 on differentiable ops
            return self.linear_fc2(gelu_tanh(self.linear_fc1(x)), residual=residual)
        return self.linear_fc2(matmul_gelu(x, self.linear_fc1.weight, self.linear_fc1.bias), residual=residual)
