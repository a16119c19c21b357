"""HIP-graph capture of a stream-ordered step (one decode token through the layers).

The reference runs its per-token decode step eagerly from Python
(models/dense.py:123-162): every op is a separate host launch, so at batch 32
the step is bound by launch overhead rather than by HBM. Every kernel of this
package is stream-ordered, allocation-free inside the C-ABI and free of host
synchronisation on the decode path, so a whole step can be captured once and
replayed as one graph launch.

Rules for a captured step:
  * inputs are static device tensors, updated in place between replays
    (token hidden states, int32 positions for `MRoPEBinding`, KV-cache lengths);
  * the step's outputs are the same tensors on every replay (`StepGraph.out`);
  * workspaces the wrappers allocate during capture live in the graph's pool
    for as long as the `StepGraph` does.
"""
from __future__ import annotations

from typing import Any, Callable, Sequence

import torch


class StepGraph:
    """Capture `fn()` (after `warmup` eager runs on a side stream) and replay it.

    `caches`: the StaticKVCaches or PagedKVCaches the step appends to,
    `tokens` rows per sequence each replay; replay() accounts for the rows on
    the host first (`reserve`, which for a paged cache assigns the pages and
    updates the block table before the launch), so a replay that would
    overflow a cache raises instead of launching.
    """

    def __init__(self, fn: Callable[[], Any], warmup: int = 2, *, caches: Sequence[Any] = (),
                 tokens: int = 1) -> None:
        if not torch.cuda.is_available():
            raise RuntimeError("StepGraph needs a GPU")
        self.fn = fn
        self.caches = list(caches)
        self.tokens = tokens
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        # Capture records the step without running it: the caches' host-side
        # lengths, which the captured forward advances, are put back after.
        # Pages the captured append writes are assigned first (a block-table
        # update is a host copy, which capture cannot record).
        for c in self.caches:
            c.prepare_append(tokens)
        saved = [c.host_state() for c in self.caches]
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = fn()
        for c, state in zip(self.caches, saved):
            c.set_host_state(state)

    def replay(self) -> Any:
        """Launch the captured step on the current stream; returns the static outputs."""
        for c in self.caches:
            c.check_reserve(self.tokens)  # raises before any cache has been advanced
        for c in self.caches:
            c.reserve(self.tokens)
        self.graph.replay()
        return self.out
