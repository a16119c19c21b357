"""CudaVisionPatchEmbed (reference modules/vision_patch.py:18-39)."""
from __future__ import annotations

import torch
from torch import nn

from ..kernels import conv3d_patch, gelu_tanh, matmul_gelu
from ..kernels.backward import needs_grad
from .linear import CudaLinear
from .norms import CudaLayerNorm


class CudaVisionPatchEmbed(nn.Module):
    """Conv3d patch embed with stride == kernel: (N, C·T·P·P) or (N, C, T, P, P) -> (N, hidden).

    weight (hidden, C, T, P, P), bias (hidden); run as an im2col GEMM (the
    input rows already are the patches).
    """

    def __init__(self, in_channels: int, hidden_size: int, patch_size: int, temporal_patch_size: int) -> None:
        super().__init__()
        self.in_channels = in_channels
        self.hidden_size = hidden_size
        self.patch_size = patch_size
        self.temporal_patch_size = temporal_patch_size
        kernel_shape = (temporal_patch_size, patch_size, patch_size)
        self.weight = nn.Parameter(torch.empty(hidden_size, in_channels, *kernel_shape))
        self.bias = nn.Parameter(torch.empty(hidden_size))
        nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)
        nn.init.zeros_(self.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() == 2:
            x = x.view(-1, self.in_channels, self.temporal_patch_size, self.patch_size, self.patch_size)
        return conv3d_patch(x, self.weight, self.bias)


class CudaVisionPatchMerger(nn.Module):
    """Spatial merge of merge x merge neighbouring patches (reference modules/vision_patch.py:42-68).

    norm (LayerNorm over the patch hidden, or over the merged hidden when
    `use_postshuffle_norm`), then linear_fc2(gelu_tanh(linear_fc1(.))) on rows
    of merge^2 consecutive tokens; fc1 and the gelu run as one GEMM.
    """

    def __init__(self, hidden_size: int, out_hidden_size: int, spatial_merge_size: int = 2,
                 use_postshuffle_norm: bool = False) -> None:
        super().__init__()
        self.hidden_size_in = hidden_size
        self.merged_hidden = hidden_size * spatial_merge_size ** 2
        self.use_postshuffle_norm = use_postshuffle_norm
        self.norm = CudaLayerNorm(self.merged_hidden if use_postshuffle_norm else hidden_size, eps=1e-6, bias=True)
        self.linear_fc1 = CudaLinear(self.merged_hidden, self.merged_hidden, bias=True)
        self.linear_fc2 = CudaLinear(self.merged_hidden, out_hidden_size, bias=True)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.use_postshuffle_norm:
            x = self.norm(x.reshape(-1, self.merged_hidden))
        else:
            x = self.norm(x).reshape(-1, self.merged_hidden)
        if needs_grad(x, *self.parameters()):  # training: fc1, gelu_tanh, fc2 on differentiable ops
            return self.linear_fc2(gelu_tanh(self.linear_fc1(x)))
        return self.linear_fc2(matmul_gelu(x, self.linear_fc1.weight, self.linear_fc1.bias))
