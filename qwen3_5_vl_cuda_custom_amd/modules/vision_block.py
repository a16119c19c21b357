"""CudaVisionBlock (reference modules/vision_block.py:13-24)."""
from __future__ import annotations

import torch
from torch import nn

from .attention import CudaVisionAttention
from .mlp import CudaVisionMLP
from .norms import CudaLayerNorm


class CudaVisionBlock(nn.Module):
    """x + Attn(LN(x)), then + MLP(LN(·)); residual adds fused into proj / linear_fc2."""

    def __init__(self, hidden_size: int, num_heads: int, intermediate_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.norm1 = CudaLayerNorm(hidden_size, eps=eps, bias=True)
        self.attn = CudaVisionAttention(hidden_size, num_heads)
        self.norm2 = CudaLayerNorm(hidden_size, eps=eps, bias=True)
        self.mlp = CudaVisionMLP(hidden_size, intermediate_size)

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *,
                cu_seqlens: torch.Tensor | None = None, max_seqlen: int | None = None) -> torch.Tensor:
        """cu_seqlens/max_seqlen: images packed into one sequence attend separately (CudaVisionAttention)."""
        x = self.attn(self.norm1(x), cos, sin, residual=x, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)
        return self.mlp(self.norm2(x), residual=x)
