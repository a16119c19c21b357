"""CudaTextDecoderLayer (reference modules/text_decoder.py:14-65)."""
from __future__ import annotations

import torch
from torch import nn

from .attention import CudaFullAttention
from .kv_cache import StaticKVCache
from .mlp import CudaSwiGLUMLP
from .moe import CudaSparseMoE
from .norms import CudaRMSNorm


class CudaTextDecoderLayer(nn.Module):
    """h = x + Attn(RMSNorm(x)); y = h + MLP(RMSNorm(h)). Returns (y, router_logits | None, (k, v)).

    Both residual adds run in the epilogues of o_proj and down_proj (or the
    MoE combine) instead of as separate passes.
    """

    def __init__(self, hidden_size: int, num_heads: int, num_kv_heads: int, head_dim: int, intermediate_size: int,
                 rms_norm_eps: float, use_moe: bool = False, num_experts: int = 0, top_k: int = 0,
                 moe_intermediate_size: int = 0, attention_bias: bool = False) -> None:
        super().__init__()
        self.input_layernorm = CudaRMSNorm(hidden_size, eps=rms_norm_eps)
        self.self_attn = CudaFullAttention(hidden_size=hidden_size, num_heads=num_heads, num_kv_heads=num_kv_heads,
                                           head_dim=head_dim, rms_norm_eps=rms_norm_eps,
                                           attention_bias=attention_bias)
        self.post_attention_layernorm = CudaRMSNorm(hidden_size, eps=rms_norm_eps)
        if use_moe:
            self.mlp = CudaSparseMoE(hidden_size=hidden_size, moe_intermediate_size=moe_intermediate_size,
                                     num_experts=num_experts, top_k=top_k)
        else:
            self.mlp = CudaSwiGLUMLP(hidden_size, intermediate_size)
        self.use_moe = use_moe

    def forward(self, x: torch.Tensor, mrope_apply, past_kv: tuple[torch.Tensor, torch.Tensor] | None = None, *,
                kv_cache: StaticKVCache | None = None):
        # Each RMSNorm is handed to the module that consumes it: at decode
        # shapes it runs inside the q/k/v (resp. gate/up) projection.
        h, new_kv = self.self_attn(x, mrope_apply, past_kv=past_kv, kv_cache=kv_cache, residual=x,
                                   input_norm=self.input_layernorm)
        if self.use_moe:
            y, router_logits = self.mlp(self.post_attention_layernorm(h), residual=h)
        else:
            y, router_logits = self.mlp(h, residual=h, input_norm=self.post_attention_layernorm), None
        return y, router_logits, new_kv
