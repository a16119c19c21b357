"""matmul: Y = X·Wᵀ + b on the gfx950 MFMA GEMM (reference kernels/matmul.py:62-77)."""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check


def matmul(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
           residual: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """nn.Linear semantics: x (..., K), weight (N, K), bias (N) -> (..., N).

    `residual` (same shape as the output) is added in the GEMM epilogue before
    the single rounding (fuses the following residual_add).
    """
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
    ws, nws = _lib.workspace(_lib.lib().q3_matmul_workspace_bytes(M, N, K, dt, 0), x.device)
    _lib.call("q3_matmul", x2.data_ptr(), w.data_ptr(), _lib.ptr(b), _lib.ptr(r2), y2.data_ptr(), M, N, K,
              x2.stride(0), w.stride(0), r2.stride(0) if r2 is not None else 0, y2.stride(0), dt,
              _lib.ptr(ws), nws, _lib.stream())
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
    wg, wu = w_gate.contiguous(), w_up.contiguous()
    M = x2.shape[0]
    y = torch.empty((*x.shape[:-1], N), dtype=x.dtype, device=x.device)
    dt = _lib.dtype_code(x.dtype)
    ws, nws = _lib.workspace(_lib.lib().q3_matmul_workspace_bytes(M, N, K, dt, 1), x.device)
    _lib.call("q3_matmul_swiglu", x2.data_ptr(), wg.data_ptr(), wu.data_ptr(), y.data_ptr(), M, N, K,
              x2.stride(0), wg.stride(0), N, dt, _lib.ptr(ws), nws, _lib.stream())
    return y
