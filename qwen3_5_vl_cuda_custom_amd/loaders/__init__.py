"""HuggingFace checkpoint loading (reference loaders/__init__.py)."""
from .hf import load_hf_weights, map_hf_name

__all__ = ["load_hf_weights", "map_hf_name"]
