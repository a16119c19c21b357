"""nn.Module drop-ins with the reference's class names, parameter names and shapes
(reference modules/__init__.py:1-28), running on libq3vl.so kernels."""
from .attention import CudaFullAttention, CudaVisionAttention
from .embedding import CudaEmbedding
from .graph import StepGraph
from .kv_cache import PagedKVCache, StaticKVCache
from .linear import CudaLinear
from .mlp import CudaSwiGLUMLP, CudaVisionMLP
from .moe import CudaSparseMoE
from .norms import CudaLayerNorm, CudaRMSNorm
from .rotary import MRoPEBinding, TextMRoPE, Vision2DRoPE
from .text_decoder import CudaTextDecoderLayer
from .vision_block import CudaVisionBlock
from .vision_patch import CudaVisionPatchEmbed, CudaVisionPatchMerger

__all__ = [
    "CudaFullAttention",
    "CudaVisionAttention",
    "CudaEmbedding",
    "CudaLinear",
    "CudaSwiGLUMLP",
    "CudaVisionMLP",
    "CudaSparseMoE",
    "CudaLayerNorm",
    "CudaRMSNorm",
    "TextMRoPE",
    "Vision2DRoPE",
    "MRoPEBinding",
    "CudaTextDecoderLayer",
    "CudaVisionBlock",
    "CudaVisionPatchEmbed",
    "CudaVisionPatchMerger",
    "PagedKVCache",
    "StaticKVCache",
    "StepGraph",
]
