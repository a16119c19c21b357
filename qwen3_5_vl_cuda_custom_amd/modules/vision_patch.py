"""CudaVisionPatchEmbed (reference modules/vision_patch.py:18-39)."""
from __future__ import annotations

import torch
from torch import nn

from ..kernels import conv3d_patch


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
