"""CudaSparseMoE (reference modules/moe.py:26-85)."""
from __future__ import annotations

import torch
from torch import nn

from ..kernels import (cuda_index_add, cuda_topk, matmul, moe_experts, moe_route, moe_router, residual_add, softmax,
                       swiglu)
from ..kernels.backward import needs_grad


class CudaSparseMoE(nn.Module):
    """Top-k routed SwiGLU experts in the HF Qwen3-VL-MoE layout.

    gate_weight (E, h); gate_up_proj (E, 2I, h) with gate rows [0, I) and up
    rows [I, 2I); down_proj (E, h, I). forward(x) -> (out, router_logits).
    Routing: softmax of the logits in fp32, top-k with the lower expert index
    winning ties, renormalised (norm_topk_prob) and cast to the input dtype.
    """

    def __init__(self, hidden_size: int, moe_intermediate_size: int, num_experts: int, top_k: int,
                 norm_topk_prob: bool = True) -> None:
        super().__init__()
        self.hidden_size = hidden_size
        self.moe_intermediate_size = moe_intermediate_size
        self.num_experts = num_experts
        self.top_k = top_k
        self.norm_topk_prob = norm_topk_prob
        self.gate_weight = nn.Parameter(torch.empty(num_experts, hidden_size))
        self.gate_up_proj = nn.Parameter(torch.empty(num_experts, 2 * moe_intermediate_size, hidden_size))
        self.down_proj = nn.Parameter(torch.empty(num_experts, hidden_size, moe_intermediate_size))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        nn.init.normal_(self.gate_weight, std=0.02)
        nn.init.normal_(self.gate_up_proj, std=0.02)
        nn.init.normal_(self.down_proj, std=0.02)

    def route(self, x_flat: torch.Tensor):
        """router_logits (T, E) in x dtype, top_idx (T, k), top_w (T, k)."""
        if x_flat.dtype == torch.bfloat16 and x_flat.shape[0] > 32:
            # prefill sizes: the logits GEMM split over K, reduced inside the routing kernel
            return moe_router(x_flat, self.gate_weight, self.top_k, self.norm_topk_prob)
        logits = matmul(x_flat, self.gate_weight)  # decode sizes: the weight-streaming GEMV
        if x_flat.dtype == torch.bfloat16:
            idx, w = moe_route(logits, self.top_k, self.norm_topk_prob)
            return logits, idx, w
        vals, idx = cuda_topk(softmax(logits.float()), self.top_k)
        if self.norm_topk_prob:
            vals = vals / vals.sum(dim=-1, keepdim=True)
        return logits, idx, vals.to(x_flat.dtype)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if needs_grad(x, residual, *self.parameters()):
            return self._forward_autograd(x, residual)
        B, S, H = x.shape
        x_flat = x.reshape(-1, H)
        logits, idx, w = self.route(x_flat)
        r_flat = residual.reshape(-1, H) if residual is not None else None
        if x.dtype == torch.bfloat16:
            out = moe_experts(x_flat, self.gate_up_proj, self.down_proj, idx, w, r_flat)
            return out.view(B, S, H), logits
        # fp32: the reference's per-expert loop on the same kernels.
        final = torch.zeros_like(x_flat)
        I = self.moe_intermediate_size
        for e in range(self.num_experts):
            mask = idx == e
            if not mask.any():
                continue
            token_idx, slot_idx = mask.nonzero(as_tuple=True)
            gu = matmul(x_flat[token_idx], self.gate_up_proj[e])
            act = swiglu(gu[:, :I].contiguous(), gu[:, I:].contiguous())
            eo = matmul(act, self.down_proj[e])
            cuda_index_add(final, (eo * w[token_idx, slot_idx, None]).to(x.dtype), token_idx)
        if r_flat is not None:
            final = residual_add(final, r_flat)
        return final.view(B, S, H), logits

    def _forward_autograd(self, x: torch.Tensor, residual: torch.Tensor | None):
        """Training: the reference's forward (modules/moe.py:54-85) on the differentiable ops: router
        GEMM, softmax of the fp32 logits, top-k, renormalise and cast, then per expert its tokens'
        gate_up GEMM, swiglu, down GEMM, the routing-weight product and the autograd form of
        index_add (a new tensor per expert)."""
        B, S, H = x.shape
        x_flat = x.reshape(-1, H)
        logits = matmul(x_flat, self.gate_weight)
        vals, idx = cuda_topk(softmax(logits.float()), self.top_k)
        if self.norm_topk_prob:
            vals = vals / vals.sum(dim=-1, keepdim=True)
        vals = vals.to(x.dtype)
        final = torch.zeros_like(x_flat)
        I = self.moe_intermediate_size
        for e in range(self.num_experts):
            token_idx, slot_idx = (idx == e).nonzero(as_tuple=True)
            if token_idx.numel() == 0:
                continue
            gu = matmul(x_flat[token_idx], self.gate_up_proj[e])
            eo = matmul(swiglu(gu[:, :I], gu[:, I:]), self.down_proj[e])
            final = cuda_index_add(final, (eo * vals[token_idx, slot_idx, None]).to(x.dtype), token_idx)
        if residual is not None:
            final = residual_add(final, residual.reshape(-1, H))
        return final.view(B, S, H), logits
