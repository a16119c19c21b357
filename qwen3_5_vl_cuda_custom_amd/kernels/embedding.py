"""embedding (reference kernels/embedding.py, csrc/embedding_op.cu:40-70): a row gather."""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check
from .backward import EmbeddingFunction, needs_grad


def embedding(ids: torch.Tensor, weight: torch.Tensor, padding_idx: int | None = None) -> torch.Tensor:
    """weight[ids] for integer ids of any shape -> (*ids.shape, dim).

    `padding_idx` only matters for initialisation and gradients (as in
    nn.Embedding); the forward gathers every id. Ids outside [0, rows) give
    zero rows and are recorded on the device (kernels.raise_device_errors),
    without synchronising with the host.
    """
    if needs_grad(weight):
        return EmbeddingFunction.apply(ids, weight, padding_idx)
    check("embedding", weight)
    if not ids.is_cuda:
        raise RuntimeError("embedding: ids must be on the GPU")
    if weight.dim() != 2:
        raise ValueError("embedding: weight must be (num_embeddings, dim)")
    flat = ids.reshape(-1).to(torch.int64).contiguous()
    w = weight.contiguous()
    rows, dim = w.shape
    out = torch.empty((flat.numel(), dim), dtype=w.dtype, device=w.device)
    _lib.call("q3_embedding", flat.data_ptr(), w.data_ptr(), out.data_ptr(), flat.numel(), rows, dim,
              _lib.dtype_code(w.dtype), _lib.status_word(w.device).data_ptr(), _lib.stream())
    return out.view(*ids.shape, dim)
