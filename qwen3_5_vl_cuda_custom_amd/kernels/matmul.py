"""matmul: Y = X·Wᵀ + b on the gfx950 MFMA GEMM (reference kernels/matmul.py:62-77)."""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check, mfma_operand, note_slow_path
from .backward import MatmulFunction, needs_grad


def _gemm_rows(op: str, K: int, *ts):
    """The row operands as the MFMA GEMM reads them (aligned copies where needed); a bf16 K that is not a
    multiple of 8 leaves only the SIMT kernel, which is reported."""
    out = [mfma_operand(op, t) for t in ts]
    if ts[0].dtype == torch.bfloat16 and K % 8:
        note_slow_path(op, f"K={K} is not a multiple of 8")
    return out


def matmul(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
           residual: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """nn.Linear semantics: x (..., K), weight (N, K), bias (N) -> (..., N).

    `residual` (same shape as the output) is added in the GEMM epilogue before
    the single rounding (fuses the following residual_add). Differentiable
    (x, weight, bias, residual) when grad mode records it.
    """
    if needs_grad(x, weight, bias, residual):
        if out is not None:
            raise ValueError("matmul: out= is not supported when autograd records the op")
        return MatmulFunction.apply(x, weight, bias, residual)
    check("matmul", x, weight, bias, residual)
    K = x.shape[-1]
    N = weight.shape[0]
    if weight.dim() != 2 or weight.shape[1] != K:
        raise ValueError(f"matmul: weight {tuple(weight.shape)} does not match x (..., {K})")
    if bias is not None and bias.shape != (N,):
        raise ValueError(f"matmul: bias {tuple(bias.shape)} != ({N},)")
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    w = weight if weight.stride(-1) == 1 else weight.contiguous()
    x2, w = _gemm_rows("matmul", K, x2, w)
    M = x2.shape[0]
    out_shape = (*x.shape[:-1], N)
    y = out if out is not None else torch.empty(out_shape, dtype=x.dtype, device=x.device)
    y2 = y.view(-1, N)
    r2 = None
    if residual is not None:
        if residual.shape != y.shape:
            raise ValueError(f"matmul: residual {tuple(residual.shape)} != output {tuple(y.shape)}")
        r2 = residual.reshape(-1, N)
        if r2.stride(-1) != 1:
            r2 = r2.contiguous()
    b = bias.contiguous() if bias is not None else None
    dt = _lib.dtype_code(x.dtype)
    ws, nws = _lib.gemm_workspace(_lib.lib().q3_matmul_workspace_bytes(M, N, K, dt, 0), x.device)
    _lib.call("q3_matmul", x2.data_ptr(), w.data_ptr(), _lib.ptr(b), _lib.ptr(r2), y2.data_ptr(), M, N, K,
              x2.stride(0), w.stride(0), r2.stride(0) if r2 is not None else 0, y2.stride(0), dt,
              _lib.ptr(ws), nws, _lib.stream())
    return y


def matmul_gelu(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """gelu_tanh(x·Wᵀ + b) in one GEMM (fc1 + gelu_tanh of modules/mlp.py:33-34 and
    modules/vision_patch.py:68), the activation applied before the single rounding."""
    check("matmul_gelu", x, weight, bias)
    K = x.shape[-1]
    N = weight.shape[0]
    if weight.dim() != 2 or weight.shape[1] != K:
        raise ValueError(f"matmul_gelu: weight {tuple(weight.shape)} does not match x (..., {K})")
    if bias is not None and bias.shape != (N,):
        raise ValueError(f"matmul_gelu: bias {tuple(bias.shape)} != ({N},)")
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    w = weight if weight.stride(-1) == 1 else weight.contiguous()
    x2, w = _gemm_rows("matmul_gelu", K, x2, w)
    y = torch.empty((*x.shape[:-1], N), dtype=x.dtype, device=x.device)
    b = bias.contiguous() if bias is not None else None
    _lib.call("q3_matmul_gelu", x2.data_ptr(), w.data_ptr(), _lib.ptr(b), y.data_ptr(), x2.shape[0], N, K,
              x2.stride(0), w.stride(0), N, _lib.dtype_code(x.dtype), _lib.stream())
    return y


def matmul_swiglu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """silu(x·W_gateᵀ)·(x·W_upᵀ) in one GEMM (the gate/up/swiglu of modules/mlp.py:19-22)."""
    check("matmul_swiglu", x, w_gate, w_up)
    K = x.shape[-1]
    N = w_gate.shape[0]
    if w_gate.shape != w_up.shape or w_gate.shape[1] != K:
        raise ValueError("matmul_swiglu: gate/up weights must both be (N, K)")
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    x2, wg, wu = _gemm_rows("matmul_swiglu", K, x2, w_gate.contiguous(), w_up.contiguous())
    M = x2.shape[0]
    y = torch.empty((*x.shape[:-1], N), dtype=x.dtype, device=x.device)
    dt = _lib.dtype_code(x.dtype)
    ws, nws = _lib.gemm_workspace(_lib.lib().q3_matmul_workspace_bytes(M, N, K, dt, 1), x.device)
    _lib.call("q3_matmul_swiglu", x2.data_ptr(), wg.data_ptr(), wu.data_ptr(), y.data_ptr(), M, N, K,
              x2.stride(0), wg.stride(0), N, dt, _lib.ptr(ws), nws, _lib.stream())
    return y


def matmul_segments(x: torch.Tensor, weights, biases=None, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Y = X·[W_0; W_1; ...]ᵀ (+ [b_0; b_1; ...]) over up to 4 weights in one GEMM.

    The weights are not concatenated: the kernel picks each output tile's
    weight matrix (q/k/v projections of modules/attention.py:82-84 in one
    launch). Returns (..., ΣN_i); the segment outputs are its column slices.
    """
    weights = list(weights)
    biases = list(biases) if biases is not None else [None] * len(weights)
    if not 1 <= len(weights) <= 4 or len(biases) != len(weights):
        raise ValueError("matmul_segments: 1 to 4 weights, one bias (or None) each")
    check("matmul_segments", x, *weights, *biases)
    K = x.shape[-1]
    ws_ = [w if w.stride(-1) == 1 and w.stride(0) == K else w.contiguous() for w in weights]
    for w, b in zip(ws_, biases):
        if w.dim() != 2 or w.shape[1] != K:
            raise ValueError(f"matmul_segments: weight {tuple(w.shape)} does not match x (..., {K})")
        if b is not None and b.shape != (w.shape[0],):
            raise ValueError(f"matmul_segments: bias {tuple(b.shape)} != ({w.shape[0]},)")
    bs = [b.contiguous() if b is not None else None for b in biases]
    ns = [w.shape[0] for w in ws_]
    N = sum(ns)
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    x2, *ws_ = _gemm_rows("matmul_segments", K, x2, *ws_)
    M = x2.shape[0]
    y = out if out is not None else torch.empty((*x.shape[:-1], N), dtype=x.dtype, device=x.device)
    y2 = y.view(-1, N)
    dt = _lib.dtype_code(x.dtype)
    n_arr = _lib.i64s(*ns)
    ws, nws = _lib.gemm_workspace(_lib.lib().q3_matmul_segments_workspace_bytes(M, n_arr, len(ns), K, dt), x.device)
    _lib.call("q3_matmul_segments", x2.data_ptr(), _lib.ptrs(*ws_),
              _lib.ptrs(*bs) if any(b is not None for b in bs) else None, n_arr, len(ns), y2.data_ptr(), M, K,
              x2.stride(0), K, y2.stride(0), dt, _lib.ptr(ws), nws, _lib.stream())
    return y


# Largest row count (tokens) of the fused RMSNorm projections: the
# weight-streaming kernel's decode shapes.
RMSNORM_MATMUL_MAX_ROWS = 32


def _norm_args(name: str, x: torch.Tensor, norm_weight: torch.Tensor, K: int):
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name}: bfloat16 only")
    if norm_weight.shape != (K,) or norm_weight.dtype != x.dtype:
        raise ValueError(f"{name}: norm weight must be ({K},) {x.dtype}")
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if x2.shape[0] > RMSNORM_MATMUL_MAX_ROWS:
        raise ValueError(f"{name}: at most {RMSNORM_MATMUL_MAX_ROWS} rows (decode shapes)")
    return mfma_operand(name, x2), mfma_operand(name, norm_weight.contiguous())


def rmsnorm_matmul_segments(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, weights,
                            biases=None) -> torch.Tensor:
    """matmul_segments(rmsnorm(x, norm_weight, eps), weights, biases) for decode
    shapes (at most 32 rows) in one launch: the rows are normalised as the
    weight-streaming kernel stages them (q3_rmsnorm_matmul_segments). Equals
    the two-op composition of modules/text_decoder.py:56 + attention.py:82-84
    to bf16 rounding."""
    weights = list(weights)
    biases = list(biases) if biases is not None else [None] * len(weights)
    if not 1 <= len(weights) <= 4 or len(biases) != len(weights):
        raise ValueError("rmsnorm_matmul_segments: 1 to 4 weights, one bias (or None) each")
    check("rmsnorm_matmul_segments", x, norm_weight, *weights, *biases)
    K = x.shape[-1]
    x2, nw = _norm_args("rmsnorm_matmul_segments", x, norm_weight, K)
    ws_ = [mfma_operand("rmsnorm_matmul_segments", w if w.stride(-1) == 1 and w.stride(0) == K else w.contiguous())
           for w in weights]
    for w, b in zip(ws_, biases):
        if w.dim() != 2 or w.shape[1] != K:
            raise ValueError(f"rmsnorm_matmul_segments: weight {tuple(w.shape)} does not match x (..., {K})")
        if b is not None and b.shape != (w.shape[0],):
            raise ValueError(f"rmsnorm_matmul_segments: bias {tuple(b.shape)} != ({w.shape[0]},)")
    bs = [b.contiguous() if b is not None else None for b in biases]
    ns = [w.shape[0] for w in ws_]
    N = sum(ns)
    M = x2.shape[0]
    y = torch.empty((*x.shape[:-1], N), dtype=x.dtype, device=x.device)
    _lib.call("q3_rmsnorm_matmul_segments", x2.data_ptr(), nw.data_ptr(), float(eps), _lib.ptrs(*ws_),
              _lib.ptrs(*bs) if any(b is not None for b in bs) else None, _lib.i64s(*ns), len(ns),
              y.data_ptr(), M, K, x2.stride(0), K, N, _lib.dtype_code(x.dtype), _lib.stream())
    return y


def rmsnorm_matmul_swiglu(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, w_gate: torch.Tensor,
                          w_up: torch.Tensor) -> torch.Tensor:
    """matmul_swiglu(rmsnorm(x, norm_weight, eps), w_gate, w_up) for decode shapes
    (at most 32 rows) in one launch (q3_rmsnorm_matmul_swiglu)."""
    check("rmsnorm_matmul_swiglu", x, norm_weight, w_gate, w_up)
    K = x.shape[-1]
    N = w_gate.shape[0]
    if w_gate.shape != w_up.shape or w_gate.shape[1] != K:
        raise ValueError("rmsnorm_matmul_swiglu: gate/up weights must both be (N, K)")
    x2, nw = _norm_args("rmsnorm_matmul_swiglu", x, norm_weight, K)
    wg, wu = (mfma_operand("rmsnorm_matmul_swiglu", w.contiguous()) for w in (w_gate, w_up))
    M = x2.shape[0]
    y = torch.empty((*x.shape[:-1], N), dtype=x.dtype, device=x.device)
    _lib.call("q3_rmsnorm_matmul_swiglu", x2.data_ptr(), nw.data_ptr(), float(eps), wg.data_ptr(), wu.data_ptr(),
              y.data_ptr(), M, N, K, x2.stride(0), wg.stride(0), N, _lib.dtype_code(x.dtype), _lib.stream())
    return y
