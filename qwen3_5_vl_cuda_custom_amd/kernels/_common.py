"""Argument checks shared by the functional ops (the reference's CHECK_INPUT, csrc/common.h:10-12)."""
from __future__ import annotations

import torch


def require_device(op: str, *tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{op}: tensors must be on the GPU (this implementation has no CPU path)")


def require_no_grad(op: str, *tensors: torch.Tensor | None) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise NotImplementedError(f"{op}: this fused / decode op has no backward; the reference's differentiable "
                                  "ops (matmul, flash_attention, rmsnorm, ... see kernels.backward) have one, or "
                                  "run under torch.no_grad() / torch.inference_mode()")


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


def _strict() -> bool:
    from ._loader import strict_mode
    return strict_mode()


def note_slow_path(op: str, reason: str) -> None:
    """A bf16 call that runs a SIMT kernel instead of the MFMA one (the layout or
    shape rules it out and no copy helps): recorded in FALLBACK_LOG, or raised
    under CUDA_QWEN3_VL_STRICT=1, like the reference's fallbacks."""
    from ._loader import record_fallback
    if _strict():
        raise RuntimeError(f"{op}: {reason} (strict mode: the MFMA kernel cannot take this call)")
    record_fallback(op, f"simt_kernel: {reason}")


def mfma_operand(op: str, t: torch.Tensor, rows_from: int = 1) -> torch.Tensor:
    """`t` as the MFMA kernels read it: a 16-byte aligned base and strides in
    multiples of 8 elements on every dim but the last (contiguous) one, from
    dim `rows_from` - 1 on. bf16 views that miss it are copied into a fresh
    contiguous buffer (the allocator aligns it) and the copy is recorded in
    FALLBACK_LOG as `aligned_copy` (raised under strict mode); the kernel then
    runs on the copy instead of dropping to its SIMT form. Other dtypes pass
    through."""
    if t.dtype != torch.bfloat16:
        return t
    if (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all(t.stride(i) % 8 == 0 for i in range(max(0, rows_from - 1), t.dim() - 1))):
        return t
    if t.shape[-1] % 8:
        return t  # a copy keeps the rows misaligned: the caller reports the SIMT path
    from ._loader import record_fallback
    if _strict():
        raise RuntimeError(f"{op}: a bf16 operand is not 16-byte aligned with strides in multiples of 8 "
                           "(strict mode: no aligned copy)")
    record_fallback(op, "aligned_copy")
    return t.contiguous() if not t.is_contiguous() else t.clone()
