"""Model assemblies over the operator layer (reference models/__init__.py)."""
from .common import CudaVisionTower
from .dense import CudaQwen3VLDenseModel
from .moe import CudaQwen3VLMoeModel

__all__ = ["CudaVisionTower", "CudaQwen3VLDenseModel", "CudaQwen3VLMoeModel"]
