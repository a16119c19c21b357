"""MI355X-native (gfx950) Qwen3-VL operator layer.

`kernels` mirrors the reference's functional op API and `modules` its
nn.Module drop-ins; both run on hand-written HIP kernels in lib/libq3vl.so
(C-ABI in include/q3vl.h), loaded through ctypes by `_lib`.
"""
from . import kernels, modules  # noqa: F401

__version__ = "0.1.0"
