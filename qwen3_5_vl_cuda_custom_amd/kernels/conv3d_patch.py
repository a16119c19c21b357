"""conv3d_patch: non-overlapping conv3d as a GEMM (reference kernels/conv3d_patch.py:17-38).

With stride == kernel size each output is a dot product of one (C, T, P, P)
patch with one filter, so (N, C·T·P·P) · (E, C·T·P·P)ᵀ + b on the MFMA GEMM.
"""
from __future__ import annotations

import torch

from .matmul import matmul


def conv3d_patch(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """x (N, C, T, H, W) with (T, H, W) == weight.shape[2:]; weight (E, C, T, H, W) -> (N, E)."""
    if x.dim() != 5 or weight.dim() != 5 or tuple(x.shape[1:]) != tuple(weight.shape[1:]):
        raise ValueError(f"conv3d_patch: input {tuple(x.shape)} must be (N, *weight.shape[1:]) "
                         f"with weight {tuple(weight.shape)}")
    N, E = x.shape[0], weight.shape[0]
    return matmul(x.reshape(N, -1), weight.reshape(E, -1), bias)
