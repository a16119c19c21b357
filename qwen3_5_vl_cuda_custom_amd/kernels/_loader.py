"""API-compatible fallback registry (reference: kernels/_loader.py:29-33, 161-269).

The reference records every CUDA->torch fallback in `FALLBACK_LOG` and can be
made strict with CUDA_QWEN3_VL_STRICT=1. This implementation has no fallback
path at all: an op whose kernel cannot run raises. The names stay importable
so code written against the reference keeps working; `FALLBACK_LOG` only ever
holds entries added through `record_fallback` by callers.
"""
from __future__ import annotations

import os
import sys

FALLBACK_LOG: list[tuple[str, str, str]] = []
_TAG = "[QWEN3-VL-HIP]"


def summarize_fallbacks() -> None:
    """Print the (caller-recorded) fallback events; the kernels themselves never fall back."""
    if not FALLBACK_LOG:
        print(f"{_TAG} no fallbacks recorded — every op ran its HIP kernel.", file=sys.stderr)
        return
    print(f"{_TAG} {len(FALLBACK_LOG)} caller-recorded fallback event(s):", file=sys.stderr)
    for op, reason, exc in FALLBACK_LOG:
        print(f"  {op}: {reason} {exc}", file=sys.stderr)


def record_fallback(op_name: str, reason: str = "not_implemented") -> None:
    FALLBACK_LOG.append((op_name, reason, ""))


def strict_mode() -> bool:
    """Reference env switch; the HIP ops always behave strictly (they raise)."""
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
