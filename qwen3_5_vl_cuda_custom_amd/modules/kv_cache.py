"""Preallocated KV cache with per-sequence lengths for the decode path.

Replaces the reference's `torch.cat` cache growth (modules/attention.py:89-92),
which re-copies the whole cache on every step, with in-place appends.
"""
from __future__ import annotations

import torch


class StaticKVCache:
    """k, v: (B, Hkv, capacity, D); lens: (B,) int32 on the device (valid rows per sequence)."""

    def __init__(self, batch: int, num_kv_heads: int, capacity: int, head_dim: int, *,
                 dtype: torch.dtype = torch.bfloat16, device: torch.device | str = "cuda",
                 lens: torch.Tensor | None = None) -> None:
        self.capacity = capacity
        self.k = torch.zeros(batch, num_kv_heads, capacity, head_dim, dtype=dtype, device=device)
        self.v = torch.zeros_like(self.k)
        self.lens = (lens.to(device=device, dtype=torch.int32).clone() if lens is not None
                     else torch.zeros(batch, dtype=torch.int32, device=device))

    @property
    def batch(self) -> int:
        return self.k.shape[0]
