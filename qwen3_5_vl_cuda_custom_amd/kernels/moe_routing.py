"""MoE routing ops (reference kernels/moe_routing.py): cuda_topk, cuda_index_add,
cuda_batched_gemm, plus the fused router and expert dispatch used by CudaSparseMoE."""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check, mfma_operand, note_slow_path
from .backward import BatchedGemmFunction, IndexAddFunction, TopKFunction, needs_grad


def cuda_topk(x: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k over the last dim: (values in x dtype, int64 indices); equal values go to the lower index."""
    if needs_grad(x):
        return TopKFunction.apply(x, k)
    check("cuda_topk", x)
    cols = x.shape[-1]
    if not 1 <= k <= cols:
        raise ValueError(f"cuda_topk: k={k} out of range for {cols} columns")
    x = x.contiguous()
    rows = x.numel() // cols
    vals = torch.empty((*x.shape[:-1], k), dtype=x.dtype, device=x.device)
    idx = torch.empty((*x.shape[:-1], k), dtype=torch.int64, device=x.device)
    _lib.call("q3_topk", x.data_ptr(), vals.data_ptr(), idx.data_ptr(), rows, cols, k, _lib.dtype_code(x.dtype),
              _lib.stream())
    return vals, idx


def cuda_index_add(target: torch.Tensor, source: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """target[index[i]] += source[i] along dim 0, in place; returns target.

    Deterministic: each target row adds its sources in ascending i in fp32,
    starting from its own value, and rounds once (torch's index_add_
    semantics). Indices must lie in [0, target.shape[0]): the kernel skips any
    other and records it on the device (see raise_device_errors); the call
    itself never synchronises with the host. When autograd records the op it
    returns a new tensor (target + the scattered sources), as the reference's
    autograd form does.
    """
    if needs_grad(target, source):
        return IndexAddFunction.apply(target, source, index)
    check("cuda_index_add", target, source)
    if index.dim() != 1 or index.shape[0] != source.shape[0] or not index.is_cuda:
        raise ValueError("cuda_index_add: index must be a 1-D device tensor with one entry per source row")
    if not target.is_contiguous():
        raise ValueError("cuda_index_add: target must be contiguous (it is updated in place)")
    if source.shape[1:] != target.shape[1:]:
        raise ValueError("cuda_index_add: source rows must match target rows")
    n_src, n_t = source.shape[0], target.shape[0]
    if n_src == 0:
        return target
    idx = index.to(torch.int64).contiguous()
    src = source.contiguous()
    D = src[0].numel()
    ws, nws = _lib.workspace(_lib.lib().q3_index_add_workspace_bytes(n_src, n_t), target.device)
    _lib.call("q3_index_add", target.data_ptr(), src.data_ptr(), idx.data_ptr(), n_src, n_t, D,
              _lib.dtype_code(target.dtype), _lib.ptr(ws), nws, _lib.status_word(target.device).data_ptr(),
              _lib.stream())
    return target


def raise_device_errors(device=None) -> None:
    """Raise for errors that device-side validation recorded since the last check (synchronises).

    cuda_index_add checks its indices on the device: a source row whose index
    lies outside [0, target rows) is skipped and flagged, with no host
    synchronisation in the op itself (so it can be captured in a HIP graph).
    """
    bits = _lib.device_status(device)
    if bits & _lib.STATUS_INDEX_OUT_OF_RANGE:
        raise IndexError("cuda_index_add: an index was out of range; its source row was skipped")


def cuda_batched_gemm(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Y[e] = X[e]·W[e]ᵀ: x (E, M, K), w (E, N, K) -> (E, M, N)."""
    if needs_grad(x, w):
        return BatchedGemmFunction.apply(x, w)
    check("cuda_batched_gemm", x, w)
    if x.dim() != 3 or w.dim() != 3 or x.shape[0] != w.shape[0] or x.shape[2] != w.shape[2]:
        raise ValueError(f"cuda_batched_gemm: x {tuple(x.shape)} and w {tuple(w.shape)} mismatch")
    E, M, K = x.shape
    N = w.shape[1]
    x, w = (mfma_operand("cuda_batched_gemm", t.contiguous()) for t in (x, w))
    if x.dtype == torch.bfloat16 and K % 8:
        note_slow_path("cuda_batched_gemm", f"K={K} is not a multiple of 8")
    y = torch.empty((E, M, N), dtype=x.dtype, device=x.device)
    _lib.call("q3_batched_gemm", x.data_ptr(), w.data_ptr(), y.data_ptr(), E, M, N, K, _lib.dtype_code(x.dtype),
              _lib.stream())
    return y


def moe_route(router_logits: torch.Tensor, top_k: int, norm_topk_prob: bool = True):
    """Fused softmax -> top-k (lowest index wins ties) -> renormalise -> bf16 (modules/moe.py:60-65).

    router_logits (T, E) bf16. Returns (top_idx int32 (T, k), top_w bf16 (T, k)).
    """
    check("moe_route", router_logits)
    if router_logits.dtype != torch.bfloat16:
        raise TypeError("moe_route: bf16 logits expected")
    lg = router_logits.contiguous()
    T, E = lg.shape
    idx = torch.empty((T, top_k), dtype=torch.int32, device=lg.device)
    w = torch.empty((T, top_k), dtype=torch.bfloat16, device=lg.device)
    _lib.call("q3_moe_route", lg.data_ptr(), idx.data_ptr(), w.data_ptr(), None, T, E, top_k,
              int(bool(norm_topk_prob)), _lib.stream())
    return idx, w


def moe_router(x: torch.Tensor, gate_weight: torch.Tensor, top_k: int, norm_topk_prob: bool = True):
    """Router logits and routing in one call (modules/moe.py:59-65), for prefill-sized T.

    x (T, H) bf16; gate_weight (E, H) bf16. The logits GEMM runs split over K into
    fp32 partials (enough tiles for every CU at T = 4096, E = 128), summed in split
    order and rounded once. Returns (logits (T, E) bf16, top_idx int32 (T, k), top_w bf16 (T, k)).
    """
    check("moe_router", x, gate_weight)
    if x.dtype != torch.bfloat16 or gate_weight.dtype != torch.bfloat16:
        raise TypeError("moe_router: bf16 inputs expected")
    xc, wc = x.contiguous(), gate_weight.contiguous()
    T, H = xc.shape
    E = wc.shape[0]
    if wc.shape[1] != H:
        raise ValueError(f"moe_router: x {tuple(xc.shape)} and gate_weight {tuple(wc.shape)} do not match")
    logits = torch.empty((T, E), dtype=torch.bfloat16, device=xc.device)
    idx = torch.empty((T, top_k), dtype=torch.int32, device=xc.device)
    w = torch.empty((T, top_k), dtype=torch.bfloat16, device=xc.device)
    ws, nws = _lib.workspace(_lib.lib().q3_moe_router_workspace_bytes(T, H, E), xc.device)
    _lib.call("q3_moe_router", xc.data_ptr(), wc.data_ptr(), logits.data_ptr(), idx.data_ptr(), w.data_ptr(), None,
              T, H, E, top_k, int(bool(norm_topk_prob)), _lib.ptr(ws), nws, _lib.stream())
    return logits, idx, w


def moe_experts(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor, top_idx: torch.Tensor,
                top_w: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
    """Dispatch, per-expert SwiGLU MLPs and combine (modules/moe.py:70-83) for routed tokens.

    x (T, H) bf16; gate_up (E, 2I, H); down (E, H, I); top_idx (T, k) int32;
    top_w (T, k) bf16. Returns (T, H) (+ residual).
    """
    check("moe_experts", x, gate_up, down, top_w, residual)
    if x.dim() != 2 or gate_up.dim() != 3 or down.dim() != 3:
        raise ValueError("moe_experts: x (T, H), gate_up (E, 2I, H), down (E, H, I)")
    T, H = x.shape
    E, I2, _ = gate_up.shape
    I = I2 // 2
    if gate_up.shape[2] != H or tuple(down.shape) != (E, H, I) or I2 % 2:
        raise ValueError(f"moe_experts: gate_up {tuple(gate_up.shape)} / down {tuple(down.shape)} do not match "
                         f"H={H}")
    if top_idx.dtype != torch.int32 or not top_idx.is_cuda or top_idx.dim() != 2 or top_idx.shape[0] != T:
        raise ValueError(f"moe_experts: top_idx must be an int32 (T={T}, k) device tensor, got {top_idx.dtype} "
                         f"{tuple(top_idx.shape)}")
    k = top_idx.shape[1]
    if tuple(top_w.shape) != (T, k):
        raise ValueError(f"moe_experts: top_w must be ({T}, {k}), got {tuple(top_w.shape)}")
    if residual is not None and tuple(residual.shape) != (T, H):
        raise ValueError(f"moe_experts: residual must be ({T}, {H})")
    x = x.contiguous()
    out = torch.empty_like(x)
    nbytes = _lib.lib().q3_moe_experts_workspace_bytes(T, H, I, E, k)
    ws, nws = _lib.workspace(nbytes, x.device)
    r = residual.contiguous() if residual is not None else None
    _lib.call("q3_moe_experts", x.data_ptr(), gate_up.contiguous().data_ptr(), down.contiguous().data_ptr(),
              top_idx.contiguous().data_ptr(), top_w.contiguous().data_ptr(), _lib.ptr(r), out.data_ptr(), T, H, I,
              E, k, _lib.ptr(ws), nws, _lib.stream())
    return out


def moe_permute(top_idx: torch.Tensor, top_w: torch.Tensor, num_experts: int):
    """The expert dispatch of CudaSparseMoE (modules/moe.py:70-76) as tables.

    top_idx (T, k) int32, top_w (T, k) bf16. Returns (offsets (E+1,) int32,
    sorted_token (T*k,) int32, sorted_w (T*k,) bf16, pos_of (T, k) int32):
    expert e's entries are rows [offsets[e], offsets[e+1]) in ascending
    (token, slot) order, the order of `(top_idx == e).nonzero()`.
    """
    check("moe_permute", top_w)
    if top_idx.dtype != torch.int32 or not top_idx.is_cuda or top_idx.dim() != 2:
        raise ValueError("moe_permute: top_idx must be an int32 (T, k) device tensor")
    if top_w.dtype != torch.bfloat16 or tuple(top_w.shape) != tuple(top_idx.shape):
        raise ValueError("moe_permute: top_w must be bf16 with top_idx's shape")
    T, k = top_idx.shape
    dev = top_idx.device
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    sorted_token = torch.empty(T * k, dtype=torch.int32, device=dev)
    sorted_w = torch.empty(T * k, dtype=torch.bfloat16, device=dev)
    pos_of = torch.full((T, k), -1, dtype=torch.int32, device=dev)
    ws, nws = _lib.workspace(_lib.lib().q3_moe_permute_workspace_bytes(T, num_experts, k), dev)
    _lib.call("q3_moe_permute", top_idx.contiguous().data_ptr(), top_w.contiguous().data_ptr(), offsets.data_ptr(),
              sorted_token.data_ptr(), sorted_w.data_ptr(), pos_of.data_ptr(), T, num_experts, k, _lib.ptr(ws), nws,
              _lib.stream())
    return offsets, sorted_token, sorted_w, pos_of
