"""Preallocated and paged KV caches with per-sequence lengths for the decode path.

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

    def check_reserve(self, n: int) -> None:
        """Raise if appending `n` rows to every sequence would overflow (nothing changes)."""
        if self.max_len + n > self.capacity:
            raise ValueError(f"StaticKVCache overflow: appending {n} row(s) to a sequence of length "
                             f"{self.max_len} exceeds the capacity {self.capacity}")

    def reserve(self, n: int) -> None:
        """Account for `n` rows about to be appended to every sequence; raises if one would overflow."""
        self.check_reserve(n)
        self.min_len += n
        self.max_len += n

    def prepare_append(self, n: int) -> None:
        """Make the next append of `n` rows capturable in a HIP graph (nothing to assign here)."""
        self.check_reserve(n)

    def host_state(self) -> tuple[int, int]:
        return self.min_len, self.max_len

    def set_host_state(self, state: tuple[int, int]) -> None:
        self.min_len, self.max_len = state


PAGED_MAX_BATCH = 1024  # the paged decode kernel's batch bound
PAGED_MAX_GROUPS = 32  # query heads per KV head in the paged decode kernel


class PagedKVCache:
    """KV cache in fixed-size pages with a per-sequence block table (no reference
    counterpart: the paged form of the decode loop's preallocated cache).

    k_pages, v_pages: (num_pages, Hkv, page_rows, D) pools; block_table:
    (B, max_pages) int32 on the device, cache row r of sequence b is row
    r % page_rows of page block_table[b, r // page_rows] (unassigned entries
    hold -1); lens: (B,) int32 on the device. page_rows is a multiple of 32 (the
    decode kernel's 32-key unit). Pages come from a host-side free list: a
    sequence gets pages as its length grows (`reserve`, `set_lens`) and gives
    them back with `release`, so ragged sequences hold only the pages they
    use. The device lengths advance inside the kernels; the host keeps every
    sequence's length (all sequences of a step grow by the same count).
    Changing the block table is a host-to-device copy, which HIP-graph capture
    cannot record: the rows a captured step will write get their pages
    beforehand (`prepare_append`).
    """

    def __init__(self, batch: int, num_kv_heads: int, head_dim: int, *, num_pages: int, max_pages: int,
                 page_rows: int = 32, dtype: torch.dtype = torch.bfloat16, device: torch.device | str = "cuda",
                 lens: torch.Tensor | list[int] | None = None) -> None:
        if page_rows < 32 or page_rows % 32:
            raise ValueError(f"PagedKVCache: page_rows must be a positive multiple of 32, got {page_rows}")
        if num_pages < 1 or max_pages < 1:
            raise ValueError("PagedKVCache: num_pages and max_pages must be positive")
        self.page_rows = page_rows
        self.max_pages = max_pages
        self.k_pages = torch.zeros(num_pages, num_kv_heads, page_rows, head_dim, dtype=dtype, device=device)
        self.v_pages = torch.zeros_like(self.k_pages)
        self.block_table = torch.full((batch, max_pages), -1, dtype=torch.int32, device=device)
        self.lens = torch.zeros(batch, dtype=torch.int32, device=device)
        self._free = list(range(num_pages - 1, -1, -1))  # stack: page 0 is handed out first
        self._pages: list[list[int]] = [[] for _ in range(batch)]
        self._host_lens = [0] * batch
        if lens is not None:
            self.set_lens(lens)

    @property
    def batch(self) -> int:
        return self.block_table.shape[0]

    def check_kernels(self, num_kv_groups: int) -> None:
        """Raise unless the paged kernels (q3_qk_norm_rope_paged, q3_decode_attention_paged) take this
        cache: bf16 rows of head_dim 128, at most PAGED_MAX_BATCH sequences and PAGED_MAX_GROUPS query
        heads per KV head. Checked before a step changes any state (lengths, pages, cache rows)."""
        D = self.k_pages.shape[-1]
        if (self.k_pages.dtype != torch.bfloat16 or D != 128 or self.batch > PAGED_MAX_BATCH
                or not 1 <= num_kv_groups <= PAGED_MAX_GROUPS):
            raise ValueError(f"PagedKVCache: the paged kernels take bf16, head_dim 128, at most {PAGED_MAX_BATCH} "
                             f"sequences and {PAGED_MAX_GROUPS} query heads per KV head (got "
                             f"{self.k_pages.dtype}, head_dim {D}, batch {self.batch}, groups {num_kv_groups})")

    @property
    def capacity(self) -> int:
        """Rows one sequence can hold (its block table's width in rows)."""
        return self.max_pages * self.page_rows

    @property
    def num_free_pages(self) -> int:
        return len(self._free)

    @property
    def min_len(self) -> int:
        return min(self._host_lens) if self._host_lens else 0

    @property
    def max_len(self) -> int:
        return max(self._host_lens) if self._host_lens else 0

    @property
    def empty(self) -> bool:
        return self.max_len == 0

    def ensure(self, rows: list[int] | int) -> None:
        """Give every sequence b pages for its rows [0, rows[b]) (an int: the same for all)."""
        want = [rows] * self.batch if isinstance(rows, int) else [int(r) for r in rows]
        if len(want) != self.batch:
            raise ValueError(f"PagedKVCache: {len(want)} row counts for a batch of {self.batch}")
        need = self._check_rows(want)
        extra = sum(max(0, n - len(p)) for n, p in zip(need, self._pages))
        if extra == 0:
            return
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("PagedKVCache: pages must be assigned before HIP-graph capture (call ensure first)")
        for b, n in enumerate(need):
            while len(self._pages[b]) < n:
                self._pages[b].append(self._free.pop())
        table = torch.full((self.batch, self.max_pages), -1, dtype=torch.int32)
        for b, pages in enumerate(self._pages):
            table[b, :len(pages)] = torch.tensor(pages, dtype=torch.int32)
        self.block_table.copy_(table)

    def _check_rows(self, want: list[int]) -> list[int]:
        """Pages each sequence needs for `want` rows; raises on overflow of a sequence or of the pool."""
        need = [-(-max(r, 0) // self.page_rows) for r in want]
        if max(need, default=0) > self.max_pages:
            raise ValueError(f"PagedKVCache overflow: {max(want)} rows exceed the capacity {self.capacity}")
        extra = sum(max(0, n - len(p)) for n, p in zip(need, self._pages))
        if extra > len(self._free):
            raise ValueError(f"PagedKVCache: {extra} more pages needed, {len(self._free)} free")
        return need

    def check_reserve(self, n: int) -> None:
        """Raise if appending `n` rows to every sequence would overflow (nothing changes)."""
        self._check_rows([L + n for L in self._host_lens])

    def prepare_append(self, n: int) -> None:
        """Assign the pages the next append of `n` rows writes, so that it can be captured in a HIP graph."""
        self.ensure([L + n for L in self._host_lens])

    def host_state(self) -> list[int]:
        return list(self._host_lens)

    def set_host_state(self, state: list[int]) -> None:
        self._host_lens = list(state)

    def set_lens(self, lens: torch.Tensor | list[int]) -> None:
        """Overwrite the per-sequence lengths; pages are assigned to cover them (never taken back here)."""
        host = [int(v) for v in torch.as_tensor(lens, dtype=torch.int64).cpu().reshape(-1)]
        if len(host) != self.batch:
            raise ValueError(f"PagedKVCache: {len(host)} lengths for a batch of {self.batch}")
        if host and (min(host) < 0 or max(host) > self.capacity):
            raise ValueError(f"PagedKVCache: lengths must lie in [0, {self.capacity}]")
        self.ensure(host)
        self.lens.copy_(torch.tensor(host, dtype=torch.int32))
        self._host_lens = host

    def reserve(self, n: int) -> None:
        """Account for `n` rows about to be appended to every sequence (pages assigned as needed)."""
        want = [L + n for L in self._host_lens]
        self.ensure(want)
        self._host_lens = want

    def release(self, b: int) -> None:
        """Return sequence b's pages to the pool and set its length to 0."""
        self._free.extend(reversed(self._pages[b]))
        self._pages[b] = []
        self.block_table[b].fill_(-1)
        self.lens[b] = 0
        self._host_lens[b] = 0

    def gather(self, rows: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Contiguous (B, Hkv, n * page_rows, D) copies of every sequence's first n = ceil(rows / page_rows)
        pages (rows past a sequence's pages are page 0's: never attended)."""
        n = max(1, -(-rows // self.page_rows))
        idx = self.block_table[:, :n].clamp(min=0).long()
        B, Hkv, P, D = self.batch, self.k_pages.shape[1], self.page_rows, self.k_pages.shape[3]

        def one(pool: torch.Tensor) -> torch.Tensor:
            return pool[idx].permute(0, 2, 1, 3, 4).reshape(B, Hkv, n * P, D)
        return one(self.k_pages), one(self.v_pages)
