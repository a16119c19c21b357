"""Argument checks shared by the functional ops (the reference's CHECK_INPUT, csrc/common.h:10-12)."""
from __future__ import annotations

import torch


def require_device(op: str, *tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{op}: tensors must be on the GPU (this implementation has no CPU path)")


def require_no_grad(op: str, *tensors: torch.Tensor | None) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise NotImplementedError(f"{op}: backward is not implemented (forward/inference only); "
                                  "run under torch.no_grad() or torch.inference_mode()")


def require_same_dtype(op: str, ref: torch.Tensor, *tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and t.dtype != ref.dtype:
            raise TypeError(f"{op}: dtype mismatch ({t.dtype} vs {ref.dtype})")


def check(op: str, *tensors: torch.Tensor | None) -> None:
    ts = [t for t in tensors if t is not None]
    require_device(op, *ts)
    require_no_grad(op, *ts)
    require_same_dtype(op, ts[0], *ts[1:])


def last_dim_contiguous(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()
