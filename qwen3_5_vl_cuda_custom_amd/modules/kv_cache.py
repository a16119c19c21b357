"""Preallocated KV cache with per-sequence lengths for the decode path.

Replaces the reference's `torch.cat` cache growth (modules/attention.py:89-92),
which re-copies the whole cache on every step, with in-place appends.
"""
from __future__ import annotations

import torch


class StaticKVCache:
    """k, v: (B, Hkv, capacity, D); lens: (B,) int32 on the device (valid rows per sequence).

    The device lengths advance inside the attention kernels, with no host
    synchronisation. The host keeps the smallest and largest length (exact:
    every append adds the same number of rows to every sequence), so an append
    past `capacity` raises before anything is launched, and a prefill knows
    whether the cache is still empty. Code that writes `lens` directly must
    call `set_lens` instead.
    """

    def __init__(self, batch: int, num_kv_heads: int, capacity: int, head_dim: int, *,
                 dtype: torch.dtype = torch.bfloat16, device: torch.device | str = "cuda",
                 lens: torch.Tensor | None = None) -> None:
        self.capacity = capacity
        self.k = torch.zeros(batch, num_kv_heads, capacity, head_dim, dtype=dtype, device=device)
        self.v = torch.zeros_like(self.k)
        self.lens = torch.zeros(batch, dtype=torch.int32, device=device)
        self.min_len = self.max_len = 0
        if lens is not None:
            self.set_lens(lens)

    @property
    def batch(self) -> int:
        return self.k.shape[0]

    @property
    def empty(self) -> bool:
        """True when every sequence has length 0."""
        return self.max_len == 0

    def set_lens(self, lens: torch.Tensor | list[int]) -> None:
        """Overwrite the per-sequence lengths (one host read of the new values)."""
        host = torch.as_tensor(lens, dtype=torch.int64).cpu().reshape(-1)
        if host.numel() != self.batch:
            raise ValueError(f"StaticKVCache: {host.numel()} lengths for a batch of {self.batch}")
        if host.numel() and (int(host.min()) < 0 or int(host.max()) > self.capacity):
            raise ValueError(f"StaticKVCache: lengths must lie in [0, {self.capacity}]")
        self.lens.copy_(host.to(torch.int32))
        self.min_len = int(host.min()) if host.numel() else 0
        self.max_len = int(host.max()) if host.numel() else 0

    def reserve(self, n: int) -> None:
        """Account for `n` rows about to be appended to every sequence; raises if one would overflow."""
        if self.max_len + n > self.capacity:
            raise ValueError(f"StaticKVCache overflow: appending {n} row(s) to a sequence of length "
                             f"{self.max_len} exceeds the capacity {self.capacity}")
        self.min_len += n
        self.max_len += n
