"""Fallback registry with the reference's names (reference: kernels/_loader.py:29-33, 161-269).

The reference records every CUDA->torch fallback in `FALLBACK_LOG` and can be
made strict with CUDA_QWEN3_VL_STRICT=1. This implementation has no torch or
CPU fallback: an op whose kernel cannot run raises. What it records instead are
the slower device paths a call can take: `aligned_copy` (a bf16 operand that
misses the MFMA kernels' 16-byte alignment, copied into an aligned buffer
first) and `simt_kernel: ...` (a bf16 call whose shape or layout only the SIMT
kernel takes). Under CUDA_QWEN3_VL_STRICT=1 those raise.
"""
from __future__ import annotations

import os
import sys

FALLBACK_LOG: list[tuple[str, str, str]] = []
_TAG = "[QWEN3-VL-HIP]"


def summarize_fallbacks() -> None:
    """Print the recorded slow-path events (aligned copies, SIMT kernels)."""
    if not FALLBACK_LOG:
        print(f"{_TAG} no fallbacks recorded — every op ran its MFMA / vector HIP kernel.", file=sys.stderr)
        return
    print(f"{_TAG} {len(FALLBACK_LOG)} fallback event(s):", file=sys.stderr)
    for op, reason, exc in FALLBACK_LOG:
        print(f"  {op}: {reason} {exc}", file=sys.stderr)


def record_fallback(op_name: str, reason: str = "not_implemented") -> None:
    FALLBACK_LOG.append((op_name, reason, ""))


def strict_mode() -> bool:
    """Reference env switch: slow device paths raise instead of being recorded."""
    return os.environ.get("CUDA_QWEN3_VL_STRICT") == "1"


def load_op(name: str, sources: list[str] | None = None, verbose: bool = False) -> bool:
    """Reference name (kernels/_loader.py:190). Every op of this package lives in the
    prebuilt libq3vl.so: True when it loads, else the load error propagates."""
    from .. import _lib
    _lib.lib()
    return True


def get_load_error(name: str) -> Exception | None:
    """Reference name (kernels/_loader.py:250): ops are never loaded per name, so there is none."""
    return None


def maybe_strict_raise(op_name: str, exc: Exception) -> None:
    """Reference name (kernels/_loader.py:258). No op here falls back, so an error always propagates."""
    raise exc
