"""Rotary ops: apply_rope / apply_mrope (reference kernels/rope.py:58-72, kernels/mrope.py:80-104)
and the fused q/k RMSNorm + mRoPE prologue used by the text attention module."""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check
from .backward import MRopeFunction, RopeFunction, needs_grad


def _bhsd_strides(t: torch.Tensor):
    return t.stride(0), t.stride(1), t.stride(2)


def _cos_dtype(c: torch.Tensor) -> int:
    return _lib.dtype_code(c.dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of x (B, H, S, D) with cos/sin (S, D_rope), (1, S, D_rope) or (B, S, D_rope).

    cos/sin are read in their own dtype (fp32 or x dtype); a batch of 1 is
    broadcast over B. Dims beyond D_rope pass through.
    """
    if needs_grad(x):
        return RopeFunction.apply(x, cos, sin)
    check("apply_rope", x)
    if not cos.is_cuda or not sin.is_cuda:
        raise RuntimeError("apply_rope: cos/sin must be on the GPU")
    if x.stride(-1) != 1:
        x = x.contiguous()
    B, H, S, D = x.shape
    Dr = cos.shape[-1]
    cos = cos.contiguous()
    sin = sin.contiguous()
    if cos.dim() == 2:
        cb = 0
    elif cos.dim() == 3 and cos.shape[0] in (1, B):
        cb = 0 if cos.shape[0] == 1 else cos.stride(0)
    else:
        raise ValueError(f"apply_rope: cos {tuple(cos.shape)} must be (S, Dr) or (B|1, S, Dr)")
    if cos.shape[-2] != S or sin.shape != cos.shape or Dr > D or Dr % 2:
        raise ValueError("apply_rope: cos/sin shape mismatch")
    y = torch.empty((B, H, S, D), dtype=x.dtype, device=x.device)
    _lib.call("q3_rope", x.data_ptr(), cos.data_ptr(), sin.data_ptr(), y.data_ptr(), B, H, S, D, Dr,
              _lib.i64s(*_bhsd_strides(x)), _lib.i64s(*_bhsd_strides(y)), cb, cos.stride(-2),
              _lib.dtype_code(x.dtype), _cos_dtype(cos), _lib.stream())
    return y


def apply_mrope(x: torch.Tensor, cos_3d: torch.Tensor, sin_3d: torch.Tensor, mrope_section: list[int]) -> torch.Tensor:
    """mRoPE of x (B, H, S, D) with cos_3d/sin_3d (3, B|1, S, D_rope) and the chunked section layout.

    Element i < D_rope/2 takes axis 0 for i < s0, axis 1 for i < s0+s1, else
    axis 2 (kernels/mrope.py:19-35), read straight from the 3-axis tables.
    """
    if needs_grad(x):
        return MRopeFunction.apply(x, cos_3d, sin_3d, mrope_section)
    check("apply_mrope", x)
    if x.stride(-1) != 1:
        x = x.contiguous()
    B, H, S, D = x.shape
    if cos_3d.dim() != 4 or cos_3d.shape[0] != 3 or sin_3d.shape != cos_3d.shape:
        raise ValueError(f"apply_mrope: cos_3d {tuple(cos_3d.shape)} must be (3, B, S, D_rope)")
    cos_3d = cos_3d.contiguous()
    sin_3d = sin_3d.contiguous()
    Dr = cos_3d.shape[-1]
    if sum(mrope_section) != Dr // 2 or cos_3d.shape[2] != S or cos_3d.shape[1] not in (1, B):
        raise ValueError("apply_mrope: mrope_section must sum to D_rope/2 and cos_3d must be (3, B|1, S, D_rope)")
    cb = 0 if cos_3d.shape[1] == 1 else cos_3d.stride(1)
    y = torch.empty((B, H, S, D), dtype=x.dtype, device=x.device)
    _lib.call("q3_mrope", x.data_ptr(), cos_3d.data_ptr(), sin_3d.data_ptr(), y.data_ptr(), B, H, S, D, Dr,
              _lib.i64s(*mrope_section), _lib.i64s(*_bhsd_strides(x)), _lib.i64s(*_bhsd_strides(y)),
              _lib.i64s(cos_3d.stride(0), cb, cos_3d.stride(2)), _lib.dtype_code(x.dtype), _cos_dtype(cos_3d),
              _lib.stream())
    return y


def qk_norm_rope(q_in, k_in, v_in, q_out, k_out, v_out, q_weight, k_weight, positions, inv_freq, mrope_section,
                 eps: float, dst_seq_offset: torch.Tensor | None = None, dst_seq_cap: int = 0) -> None:
    """Fused per-head RMSNorm (optional) + mRoPE of q and k, and copy of v (optional).

    All six tensors are (B, S, H, D) views (any strides, D contiguous);
    positions (3, B, S) int32 and inv_freq (D/2) fp32 on the device.
    dst_seq_offset (B,) int32 shifts the sequence index of the k/v outputs
    (cache append); rows landing at index >= dst_seq_cap (if > 0) are dropped.
    """
    B, S, Hq, D = q_in.shape
    Hkv = k_in.shape[2]
    # The kernel reads positions[(axis * B + b) * S + s] and inv_freq[0, D/2):
    # anything else would be read out of bounds on the device.
    if (positions.dtype != torch.int32 or not positions.is_cuda or tuple(positions.shape) != (3, B, S)
            or not positions.is_contiguous()):
        raise ValueError(f"qk_norm_rope: positions must be a contiguous int32 (3, {B}, {S}) device tensor, got "
                         f"{positions.dtype} {tuple(positions.shape)}")
    if inv_freq.dtype != torch.float32 or not inv_freq.is_cuda or inv_freq.numel() != D // 2:
        raise ValueError(f"qk_norm_rope: inv_freq must be a float32 ({D // 2},) device tensor")
    if dst_seq_offset is not None and (dst_seq_offset.dtype != torch.int32 or not dst_seq_offset.is_cuda
                                       or tuple(dst_seq_offset.shape) != (B,) or not dst_seq_offset.is_contiguous()):
        raise ValueError(f"qk_norm_rope: dst_seq_offset must be a contiguous int32 ({B},) device tensor")
    if tuple(k_in.shape) != (B, S, Hkv, D) or tuple(q_out.shape) != (B, S, Hq, D):
        raise ValueError("qk_norm_rope: q/k views must be (B, S, H, D) with matching B, S and D")
    if sum(mrope_section) * 2 != D:
        raise ValueError(f"qk_norm_rope: mrope_section {list(mrope_section)} must sum to D/2 = {D // 2}")
    ts = [q_in, k_in, v_in, q_out, k_out, v_out]
    strides = []
    for t in ts:
        if t is None:
            strides += [0, 0, 0]
        else:
            if t.stride(-1) != 1:
                raise ValueError("qk_norm_rope: the head dim must be contiguous")
            strides += [t.stride(0), t.stride(1), t.stride(2)]
    _lib.call("q3_qk_norm_rope", q_in.data_ptr(), k_in.data_ptr(), _lib.ptr(v_in), q_out.data_ptr(),
              k_out.data_ptr(), _lib.ptr(v_out), _lib.ptr(q_weight), _lib.ptr(k_weight), positions.data_ptr(),
              inv_freq.data_ptr(), _lib.ptr(dst_seq_offset), int(dst_seq_cap), B, S, Hq, Hkv, D,
              _lib.i64s(*mrope_section),
              float(eps), _lib.i64s(*strides), _lib.dtype_code(q_in.dtype), _lib.stream())


def qk_norm_rope_paged(q_in, k_in, v_in, q_out, k_pages, v_pages, q_weight, k_weight, positions, inv_freq,
                       mrope_section, eps: float, block_table: torch.Tensor, kv_lens: torch.Tensor,
                       status: torch.Tensor | None = None) -> None:
    """qk_norm_rope with the k/v rows appended to a paged cache (no reference counterpart).

    q_in/k_in/v_in/q_out (B, S, H, D) views as for qk_norm_rope; k_pages/v_pages
    (num_pages, Hkv, page_rows, D) pools; block_table (B, max_pages) int32 and
    kv_lens (B,) int32 on the device: the rows go to cache rows kv_lens[b] + s.
    A page id outside the pool drops the row and sets bit 1 of `status`
    (default: the device's status word).
    """
    B, S, Hq, D = q_in.shape
    Hkv = k_in.shape[2]
    if (positions.dtype != torch.int32 or not positions.is_cuda or tuple(positions.shape) != (3, B, S)
            or not positions.is_contiguous()):
        raise ValueError(f"qk_norm_rope_paged: positions must be a contiguous int32 (3, {B}, {S}) device tensor")
    if inv_freq.dtype != torch.float32 or not inv_freq.is_cuda or inv_freq.numel() != D // 2:
        raise ValueError(f"qk_norm_rope_paged: inv_freq must be a float32 ({D // 2},) device tensor")
    if (block_table.dtype != torch.int32 or not block_table.is_cuda or block_table.dim() != 2
            or block_table.shape[0] != B or not block_table.is_contiguous()):
        raise ValueError("qk_norm_rope_paged: block_table must be a contiguous int32 (B, max_pages) device tensor")
    if kv_lens.dtype != torch.int32 or not kv_lens.is_cuda or kv_lens.shape != (B,) or kv_lens.stride(0) != 1:
        raise ValueError("qk_norm_rope_paged: kv_lens must be a contiguous int32 (B,) device tensor")
    if tuple(k_in.shape) != (B, S, Hkv, D) or tuple(q_out.shape) != (B, S, Hq, D):
        raise ValueError("qk_norm_rope_paged: q/k views must be (B, S, H, D) with matching B, S and D")
    if k_pages.shape != v_pages.shape or k_pages.shape[1] != Hkv or k_pages.shape[3] != D:
        raise ValueError(f"qk_norm_rope_paged: pages {tuple(k_pages.shape)} for Hkv={Hkv}, D={D}")
    if sum(mrope_section) * 2 != D:
        raise ValueError(f"qk_norm_rope_paged: mrope_section {list(mrope_section)} must sum to D/2 = {D // 2}")
    strides = []
    for t in [q_in, k_in, v_in, q_out]:
        if t.stride(-1) != 1:
            raise ValueError("qk_norm_rope_paged: the head dim must be contiguous")
        strides += [t.stride(0), t.stride(1), t.stride(2)]
    for t in [k_pages, v_pages]:
        if t.stride(-1) != 1:
            raise ValueError("qk_norm_rope_paged: the pages' head dim must be contiguous")
        strides += [t.stride(0), t.stride(2), t.stride(1)]  # (page, row, head)
    st = status if status is not None else _lib.status_word(q_in.device)
    _lib.call("q3_qk_norm_rope_paged", q_in.data_ptr(), k_in.data_ptr(), v_in.data_ptr(), q_out.data_ptr(),
              k_pages.data_ptr(), v_pages.data_ptr(), _lib.ptr(q_weight), _lib.ptr(k_weight), positions.data_ptr(),
              inv_freq.data_ptr(), block_table.data_ptr(), block_table.shape[1], k_pages.shape[2], k_pages.shape[0],
              kv_lens.data_ptr(), B, S, Hq, Hkv, D, _lib.i64s(*mrope_section), float(eps), _lib.i64s(*strides),
              _lib.dtype_code(q_in.dtype), st.data_ptr(), _lib.stream())
