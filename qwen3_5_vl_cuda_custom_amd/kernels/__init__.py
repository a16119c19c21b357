"""Functional ops with the reference's names and signatures (reference kernels/__init__.py:1-45),
each backed by a hand-written gfx950 HIP kernel of libq3vl.so. GPU tensors only; no fallback.
The ops the reference wraps in torch.autograd.Function are differentiable here too (kernels/backward.py)."""
from ._loader import FALLBACK_LOG, record_fallback, strict_mode, summarize_fallbacks
from .conv3d_patch import conv3d_patch
from .cross_entropy import cross_entropy
from .elementwise import gelu_tanh, residual_add, sigmoid_mul, swiglu
from .embedding import embedding
from .flash_attention import (decode_attention, decode_attention_paged, flash_attention, flash_attention_cache,
                              flash_attention_cache_paged,
                              flash_attention_varlen, qk_norm_rope_attention, qk_norm_rope_attention_ok)
from .matmul import (RMSNORM_MATMUL_MAX_ROWS, matmul, matmul_gelu, matmul_segments, matmul_swiglu,
                     rmsnorm_matmul_segments, rmsnorm_matmul_swiglu)
from .moe_routing import (cuda_batched_gemm, cuda_index_add, cuda_topk, moe_experts, moe_permute, moe_route,
                          moe_router, raise_device_errors)
from .norms import layernorm, rmsnorm, softmax
from .rotary import apply_mrope, apply_rope, qk_norm_rope, qk_norm_rope_paged
from .vision import vision_pos_embed, vision_rope_tables

__all__ = [
    "FALLBACK_LOG",
    "summarize_fallbacks",
    "record_fallback",
    "strict_mode",
    "apply_mrope",
    "apply_rope",
    "conv3d_patch",
    "cross_entropy",
    "cuda_batched_gemm",
    "cuda_index_add",
    "cuda_topk",
    "embedding",
    "flash_attention",
    "gelu_tanh",
    "layernorm",
    "matmul",
    "residual_add",
    "rmsnorm",
    "sigmoid_mul",
    "softmax",
    "swiglu",
    # additions beyond the reference API (fused / decode / MoE dispatch paths)
    "decode_attention",
    "decode_attention_paged",
    "flash_attention_cache",
    "flash_attention_cache_paged",
    "flash_attention_varlen",
    "matmul_gelu",
    "vision_rope_tables",
    "vision_pos_embed",
    "matmul_segments",
    "matmul_swiglu",
    "rmsnorm_matmul_segments",
    "rmsnorm_matmul_swiglu",
    "RMSNORM_MATMUL_MAX_ROWS",
    "moe_experts",
    "moe_route",
    "moe_router",
    "moe_permute",
    "raise_device_errors",
    "qk_norm_rope",
    "qk_norm_rope_paged",
    "qk_norm_rope_attention",
    "qk_norm_rope_attention_ok",
]
