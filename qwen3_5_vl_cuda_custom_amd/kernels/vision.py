"""Vision-tower glue on the GPU: 2D rotary tables and position-embedding interpolation
(reference models/common.py:85-174), computed from the images' (t, h, w) grids."""
from __future__ import annotations

import ctypes

import torch

from .. import _lib
from ._common import check


def image_table(grid_thw, merge: int, device) -> tuple[torch.Tensor, ctypes.Array, int]:
    """(n_img, 4) int32 rows (t, h, w, first token) on the device and on the host, and the token total.

    grid_thw: an (n, 3) tensor or a list of (t, h, w) in patch units; h and w
    must be multiples of `merge`.
    """
    rows = [tuple(int(v) for v in r) for r in (grid_thw.tolist() if torch.is_tensor(grid_thw) else grid_thw)]
    flat, first = [], 0
    for t, h, w in rows:
        if t < 1 or h < 1 or w < 1 or h % merge or w % merge:
            raise ValueError(f"image grid {(t, h, w)}: sizes must be positive, h and w multiples of {merge}")
        flat += [t, h, w, first]
        first += t * h * w
    host = (ctypes.c_int * len(flat))(*flat)
    dev = torch.tensor(flat, dtype=torch.int32).to(device, non_blocking=False)
    return dev, host, first


def vision_rope_tables(grid_thw, merge: int, inv_freq: torch.Tensor, head_dim: int):
    """cos, sin (total, head_dim) fp32: row/column angles per patch (models/common.py:85-120, 192-195)."""
    if not inv_freq.is_cuda or inv_freq.dtype != torch.float32 or inv_freq.numel() != head_dim // 4:
        raise ValueError(f"vision_rope_tables: inv_freq must be float32 ({head_dim // 4},) on the GPU")
    dev_tab, host_tab, total = image_table(grid_thw, merge, inv_freq.device)
    cos = torch.empty((total, head_dim), dtype=torch.float32, device=inv_freq.device)
    sin = torch.empty_like(cos)
    _lib.call("q3_vision_rope_tables", dev_tab.data_ptr(), ctypes.addressof(host_tab), len(host_tab) // 4, merge,
              head_dim, inv_freq.contiguous().data_ptr(), cos.data_ptr(), sin.data_ptr(), _lib.stream())
    return cos, sin


def vision_pos_embed(x: torch.Tensor, table: torch.Tensor, grid_thw, merge: int, *,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """x + bilinear interpolation of the learned (G*G, hidden) position table at every
    patch (models/common.py:122-174), in token order; `out` may be x itself."""
    check("vision_pos_embed", x, table)
    side = int(round(table.shape[0] ** 0.5))
    if side * side != table.shape[0] or table.shape[1] != x.shape[-1]:
        raise ValueError(f"vision_pos_embed: table {tuple(table.shape)} must be (G*G, {x.shape[-1]})")
    dev_tab, host_tab, total = image_table(grid_thw, merge, x.device)
    if x.dim() != 2 or x.shape[0] != total or not x.is_contiguous():
        raise ValueError(f"vision_pos_embed: x must be contiguous ({total}, hidden)")
    y = out if out is not None else torch.empty_like(x)
    _lib.call("q3_vision_pos_embed", dev_tab.data_ptr(), ctypes.addressof(host_tab), len(host_tab) // 4, merge, side,
              table.contiguous().data_ptr(), x.data_ptr(), y.data_ptr(), x.shape[1], _lib.dtype_code(x.dtype),
              _lib.stream())
    return y
