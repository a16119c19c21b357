"""Model configuration (reference configs/__init__.py)."""
from .config import MoETextConfig, Qwen3VLConfig, TextConfig, VisionConfig

__all__ = ["VisionConfig", "TextConfig", "MoETextConfig", "Qwen3VLConfig"]
