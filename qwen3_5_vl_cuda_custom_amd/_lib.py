"""ctypes binding of libq3vl.so (the C-ABI declared in include/q3vl.h).

The library is loaded from `qwen3_5_vl_cuda_custom_amd/lib/libq3vl.so`, built
ahead of time by `qwen3_5_vl_cuda_custom_amd.build`. There is no fallback:
if the library is missing, every op raises.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libq3vl.so"

Q3_F32 = 0
Q3_BF16 = 1

_i64p = POINTER(c_int64)
_i32p = c_void_p
_f32p = c_void_p
_V = c_void_p
_I = c_int64

# name -> (restype, argtypes)
_SIGS: dict[str, tuple] = {
    "q3_abi_version": (c_int, []),
    "q3_error_string": (c_char_p, [c_int]),
    "q3_matmul_workspace_bytes": (c_int64, [_I, _I, _I, c_int, c_int]),
    "q3_matmul": (c_int, [_V, _V, _V, _V, _V, _I, _I, _I, _I, _I, _I, _I, c_int, _V, _I, _V]),
    "q3_matmul_swiglu": (c_int, [_V, _V, _V, _V, _I, _I, _I, _I, _I, _I, c_int, _V, _I, _V]),
    "q3_matmul_gelu": (c_int, [_V, _V, _V, _V, _I, _I, _I, _I, _I, _I, c_int, _V]),
    "q3_matmul_segments_workspace_bytes": (c_int64, [_I, _i64p, _I, _I, c_int]),
    "q3_matmul_segments": (c_int, [_V, _V, _V, _i64p, _I, _V, _I, _I, _I, _I, _I, c_int, _V, _I, _V]),
    "q3_rmsnorm_matmul_segments": (c_int, [_V, _V, c_float, _V, _V, _i64p, _I, _V, _I, _I, _I, _I, _I, c_int, _V]),
    "q3_rmsnorm_matmul_swiglu": (c_int, [_V, _V, c_float, _V, _V, _V, _I, _I, _I, _I, _I, _I, c_int, _V]),
    "q3_batched_gemm": (c_int, [_V, _V, _V, _I, _I, _I, _I, c_int, _V]),
    "q3_residual_add": (c_int, [_V, _V, _V, _I, c_int, _V]),
    "q3_swiglu": (c_int, [_V, _V, _V, _I, c_int, _V]),
    "q3_gelu_tanh": (c_int, [_V, _V, _I, c_int, _V]),
    "q3_rmsnorm": (c_int, [_V, _V, _V, _I, _I, c_float, c_int, _V]),
    "q3_layernorm": (c_int, [_V, _V, _V, _V, _I, _I, c_float, c_int, _V]),
    "q3_softmax": (c_int, [_V, _V, _I, _I, c_int, _V]),
    "q3_topk": (c_int, [_V, _V, _V, _I, _I, _I, c_int, _V]),
    "q3_rope": (c_int, [_V, _V, _V, _V, _I, _I, _I, _I, _I, _i64p, _i64p, _I, _I, c_int, c_int, _V]),
    "q3_mrope": (c_int, [_V, _V, _V, _V, _I, _I, _I, _I, _I, _i64p, _i64p, _i64p, _i64p, c_int, c_int, _V]),
    "q3_qk_norm_rope": (c_int, [_V, _V, _V, _V, _V, _V, _V, _V, _i32p, _f32p, _i32p, _I, _I, _I, _I, _I, _I,
                                _i64p, c_float, _i64p, c_int, _V]),
    "q3_flash_attention": (c_int, [_V, _V, _V, _V, _f32p, _I, _I, _I, _I, _I, _I, _i64p, c_float, c_int, c_int,
                                   _V]),
    "q3_qk_norm_rope_attention_workspace_bytes": (c_int64, [_I, _I, _I]),
    "q3_qk_norm_rope_attention": (c_int, [_V, _V, _V, _V, _V, _V, _i32p, _f32p, _I, _I, _I, _I, _I, _i64p, c_float,
                                          _i64p, c_float, c_int, c_int, _V, _I, _V]),
    "q3_flash_attention_varlen": (c_int, [_V, _V, _V, _V, _i32p, _I, _I, _I, _I, _I, _I, _i64p, c_float, c_int,
                                          c_int, _V]),
    "q3_flash_attention_cache": (c_int, [_V, _V, _V, _i32p, _V, _I, _I, _I, _I, _I, _I, _i64p, c_float, c_int,
                                         c_int, _V]),
    "q3_flash_attention_cache_paged": (c_int, [_V, _V, _V, _i32p, _I, _I, _I, _i32p, _V, _I, _I, _I, _I, _I, _i64p,
                                               c_float, c_int, c_int, _i32p, _V]),
    "q3_decode_attention_workspace_bytes": (c_int64, [_I, _I, _I, _I, _I]),
    "q3_decode_attention": (c_int, [_V, _V, _V, _i32p, _V, _I, _I, _I, _I, _I, _i64p, c_float, c_int, _V, _I, _V]),
    "q3_decode_attention_step": (c_int, [_V, _V, _V, _i32p, _V, _I, _I, _I, _I, _I, _i64p, c_float, c_int, _V, _I,
                                         _V]),
    "q3_qk_norm_rope_paged": (c_int, [_V, _V, _V, _V, _V, _V, _V, _V, _i32p, _f32p, _i32p, _I, _I, _I, _i32p, _I,
                                      _I, _I, _I, _I, _i64p, c_float, _i64p, c_int, _i32p, _V]),
    "q3_decode_attention_paged": (c_int, [_V, _V, _V, _i32p, _I, _I, _I, _i32p, c_int, _V, _I, _I, _I, _I, _i64p,
                                          c_float, c_int, _V, _I, _i32p, _V]),
    "q3_decode_attention_step_noalloc_max_bytes": (c_int64, []),
    "q3_decode_attention_step_noalloc": (c_int, [_V, _V, _V, _i32p, _V, _I, _I, _I, _I, _I, _i64p, c_float, c_int,
                                                 _V]),
    "q3_embedding": (c_int, [_V, _V, _V, _I, _I, _I, c_int, _i32p, _V]),
    "q3_vision_rope_tables": (c_int, [_i32p, _i32p, _I, _I, _I, _f32p, _f32p, _f32p, _V]),
    "q3_vision_pos_embed": (c_int, [_i32p, _i32p, _I, _I, _I, _V, _V, _V, _I, c_int, _V]),
    "q3_moe_route": (c_int, [_V, _i32p, _V, _f32p, _I, _I, _I, c_int, _V]),
    "q3_moe_router_workspace_bytes": (c_int64, [_I, _I, _I]),
    "q3_moe_router": (c_int, [_V, _V, _V, _i32p, _V, _f32p, _I, _I, _I, _I, c_int, _V, _I, _V]),
    "q3_moe_experts_workspace_bytes": (c_int64, [_I, _I, _I, _I, _I]),
    "q3_moe_experts": (c_int, [_V, _V, _V, _i32p, _V, _V, _V, _I, _I, _I, _I, _I, _V, _I, _V]),
    "q3_moe_permute_workspace_bytes": (c_int64, [_I, _I, _I]),
    "q3_moe_permute": (c_int, [_i32p, _V, _i32p, _i32p, _V, _i32p, _I, _I, _I, _V, _I, _V]),
    "q3_index_add_workspace_bytes": (c_int64, [_I, _I]),
    "q3_index_add": (c_int, [_V, _V, _V, _I, _I, _I, c_int, _V, _I, _i32p, _V]),
    # the rest of the op namespace and the backward entry points (train.hip, attention_bwd.hip)
    "q3_sigmoid_mul": (c_int, [_V, _V, _V, _I, c_int, _V]),
    "q3_sigmoid_mul_backward": (c_int, [_V, _V, _V, _V, _V, _I, c_int, _V]),
    "q3_swiglu_backward": (c_int, [_V, _V, _V, _V, _V, _I, c_int, _V]),
    "q3_gelu_tanh_backward": (c_int, [_V, _V, _V, _I, c_int, _V]),
    "q3_softmax_backward": (c_int, [_V, _V, _V, _I, _I, c_int, _V]),
    "q3_norm_backward_workspace_bytes": (c_int64, [_I, _I]),
    "q3_rmsnorm_backward": (c_int, [_V, _V, _V, _V, _V, _I, _I, c_float, c_int, _V, _I, _V]),
    "q3_layernorm_backward": (c_int, [_V, _V, _V, _V, _V, _V, _I, _I, c_float, c_int, _V, _I, _V]),
    "q3_cross_entropy": (c_int, [_V, _V, _f32p, _f32p, _f32p, _i32p, _I, _I, _I, c_int, _i32p, _V]),
    "q3_cross_entropy_backward": (c_int, [_V, _V, _f32p, _f32p, _i32p, _V, _I, _I, _I, c_int, _V]),
    "q3_topk_backward": (c_int, [_V, _V, _V, _I, _I, _I, c_int, _V]),
    "q3_transpose": (c_int, [_V, _V, _I, _I, _I, c_int, _V]),
    "q3_matmul_backward_workspace_bytes": (c_int64, [_I, _I, _I, c_int]),
    "q3_matmul_backward": (c_int, [_V, _V, _V, _V, _V, _V, _I, _I, _I, c_int, _V, _I, _V, _I, _V]),
    "q3_batched_gemm_backward_workspace_bytes": (c_int64, [_I, _I, _I, _I, c_int]),
    "q3_batched_gemm_backward": (c_int, [_V, _V, _V, _V, _V, _I, _I, _I, _I, c_int, _V, _I, _V]),
    "q3_flash_attention_backward_workspace_bytes": (c_int64, [_I, _I, _I]),
    "q3_flash_attention_backward": (c_int, [_V, _V, _V, _V, _f32p, _V, _V, _V, _V, _I, _I, _I, _I, _I, _I, c_float,
                                            c_int, c_int, _V, _I, _V]),
}

EXPORTED = tuple(_SIGS)

_lib: ctypes.CDLL | None = None


class Q3Error(RuntimeError):
    """A libq3vl entry point returned a non-zero status."""

    def __init__(self, op: str, code: int, msg: str):
        super().__init__(f"{op} failed: {msg} (status {code})")
        self.op = op
        self.code = code


def lib() -> ctypes.CDLL:
    """Load libq3vl.so once and bind every entry point's signature."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m qwen3_5_vl_cuda_custom_amd.build` "
                "(there is no fallback path)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def error_string(code: int) -> str:
    return lib().q3_error_string(code).decode()


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise Q3Error(name, rc, error_string(rc))


def i64s(*vals) -> ctypes.Array:
    return (c_int64 * len(vals))(*[int(v) for v in vals])


def ptrs(*ts) -> ctypes.Array:
    """A C array of device pointers (NULL for None)."""
    return (c_void_p * len(ts))(*[None if t is None else t.data_ptr() for t in ts])


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return Q3_BF16
    if dt == torch.float32:
        return Q3_F32
    raise TypeError(f"unsupported dtype {dt}: the kernels take bfloat16 or float32")


def workspace(nbytes: int, device: torch.device) -> tuple[torch.Tensor | None, int]:
    """A device scratch buffer of at least `nbytes` (None when 0)."""
    if nbytes <= 0:
        return None, 0
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device), int(nbytes)


# Per-device GEMM workspaces: the decode GEMVs' (M <= 32) and the fp32 partial
# planes of a prefill-sized GEMM split over K. They start zero-filled: their
# first 16 KiB are tile counters that every call leaves at zero again (the
# planes lie behind them). A larger request allocates a new buffer; the old
# ones are kept, because captured HIP graphs may still point at them. Calls on
# different streams that run at the same time must not share one: these serve
# stream-ordered work (a layer's GEMMs, the decode step).
_gemm_ws: dict[tuple[str, int | None], list[torch.Tensor]] = {}


def gemm_workspace(nbytes: int, device: torch.device) -> tuple[torch.Tensor | None, int]:
    """The zero-initialised, persistent workspace of the GEMM entry points."""
    if nbytes <= 0:
        return None, 0
    dev = torch.device(device)
    key = (dev.type, dev.index if dev.index is not None else torch.cuda.current_device())
    bufs = _gemm_ws.setdefault(key, [])
    if not bufs or bufs[-1].numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("gemm_workspace: first use of this GEMM size inside HIP-graph capture; run the "
                               "step once eagerly before capturing it (StepGraph does)")
        size = max(int(nbytes), 2 * bufs[-1].numel() if bufs else 0, 16 << 20)
        bufs.append(torch.zeros(size, dtype=torch.uint8, device=dev))
    buf = bufs[-1]
    return buf, buf.numel()


# Per-device sticky status words (one int32 each, zero-initialised): kernels
# that validate device-side data (index_add's indices) set bits here instead
# of synchronising with the host. `device_status` reads and clears them.
_status: dict[int, torch.Tensor] = {}

STATUS_INDEX_OUT_OF_RANGE = 1
STATUS_BAD_PAGE = 2  # a paged-cache block table named a page outside the pool


def status_word(device: torch.device) -> torch.Tensor:
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    t = _status.get(idx)
    if t is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("status_word: first use on this device inside HIP-graph capture; run the op once "
                               "eagerly before capturing it")
        t = _status[idx] = torch.zeros(1, dtype=torch.int32, device=dev)
    return t


def device_status(device: torch.device | str | None = None, clear: bool = True) -> int:
    """The bits set on `device` since the last clear (synchronises with the device)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    t = _status.get(dev.index if dev.index is not None else torch.cuda.current_device())
    if t is None:
        return 0
    v = int(t.item())
    if clear and v:
        t.zero_()
    return v
