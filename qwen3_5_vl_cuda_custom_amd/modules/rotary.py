"""Rotary helpers: Vision2DRoPE and TextMRoPE (reference modules/rotary.py:9-59)."""
from __future__ import annotations

import torch
from torch import nn

from ..kernels import apply_mrope, apply_rope, qk_norm_rope
from ..kernels.backward import needs_grad


def rotary_inv_freq(dim: int, theta: float, device=None) -> torch.Tensor:
    """inv_freq = 1 / theta^(arange(0, dim, 2) / dim) in fp32 (reference modules/rotary.py:19, 43)."""
    return 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float32, device=device) / dim))


class _FP32Freqs(nn.Module):
    """Keeps the `inv_freq` buffer in fp32 through `.to(dtype)` / `.half()` casts of a model:
    the rotation angles are computed from it in fp32 by the kernels."""

    _freq_dim: int
    _freq_theta: float

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse)
        if self.inv_freq.dtype != torch.float32:
            self.inv_freq = rotary_inv_freq(self._freq_dim, self._freq_theta, self.inv_freq.device)
        return self


class Vision2DRoPE(_FP32Freqs):
    """Vision rotary embedding; forward(seqlen) -> freqs (S, dim//2) (reference modules/rotary.py:9-31)."""

    def __init__(self, dim: int, theta: float = 10000.0) -> None:
        super().__init__()
        self.dim = dim
        self.theta = theta
        self._freq_dim, self._freq_theta = dim, theta
        self.register_buffer("inv_freq", rotary_inv_freq(dim, theta), persistent=False)

    def forward(self, seqlen: int) -> torch.Tensor:
        seq = torch.arange(seqlen, device=self.inv_freq.device, dtype=self.inv_freq.dtype)
        return torch.outer(seq, self.inv_freq)

    @staticmethod
    def apply(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
        """RoPE of q/k (B, H, S, D)."""
        return apply_rope(q, cos, sin), apply_rope(k, cos, sin)


class MRoPEBinding:
    """`mrope_apply` callable for a fixed set of positions, as passed to the attention modules.

    Calling it, binding(q, k), rotates q and k like the reference's
    `lambda q, k: rotary.apply(q, k, position_ids)` (models/dense.py:68). The
    attention module recognises a binding and fuses the rotation with the
    q/k RMSNorm in one kernel straight from the integer positions.
    """

    def __init__(self, rope: "TextMRoPE", position_ids: torch.Tensor) -> None:
        self.rope = rope
        self.position_ids = position_ids
        self._pos32: torch.Tensor | None = None

    def positions_int32(self, device: torch.device, batch: int | None = None, seq: int | None = None) -> torch.Tensor:
        """(3, B, S) int32 positions on `device`, checked against the batch and
        sequence length of the tokens they rotate. (3, 1, S) positions are
        broadcast over the batch (a copy), as TextMRoPE.apply and the
        reference's cos/sin tables do; any other shape raises. An int32
        contiguous (3, B, S) device tensor passed at construction is used as is,
        so in-place updates of it reach the kernels (a captured decode step
        reads its positions from there)."""
        pid = self.position_ids
        if pid.dim() != 3 or pid.shape[0] != 3:
            raise ValueError(f"mRoPE positions must be (3, B, S), got {tuple(pid.shape)}")
        if seq is not None and pid.shape[2] != seq:
            raise ValueError(f"mRoPE positions cover {pid.shape[2]} tokens, the input has {seq}")
        if batch is not None and pid.shape[1] not in (1, batch):
            raise ValueError(f"mRoPE positions have batch {pid.shape[1]}, the input has {batch}")
        want_b = batch if batch is not None else pid.shape[1]
        p = self._pos32
        if p is None or p.device != torch.device(device) or p.shape[1] != want_b:
            p = pid.to(device=device, dtype=torch.int32)
            if p.shape[1] != want_b:
                p = p.expand(3, want_b, p.shape[2])
            self._pos32 = p = p.contiguous()
        return p

    def __call__(self, q: torch.Tensor, k: torch.Tensor):
        return self.rope.apply(q, k, self.position_ids)


class TextMRoPE(_FP32Freqs):
    """Text mRoPE: 3D positions (T, H, W) over the head dim by `mrope_section` (reference modules/rotary.py:34-59)."""

    def __init__(self, dim: int, theta: float = 500000.0, mrope_section: list[int] | None = None) -> None:
        super().__init__()
        self.dim = dim
        self.theta = theta
        self.mrope_section = list(mrope_section or [24, 20, 20])
        self._freq_dim, self._freq_theta = dim, theta
        self.register_buffer("inv_freq", rotary_inv_freq(dim, theta), persistent=False)

    def compute_cos_sin(self, position_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """position_ids (3, B, S) -> cos/sin (3, B, S, dim) fp32 (reference modules/rotary.py:46-55)."""
        freqs = position_ids.float().unsqueeze(-1) * self.inv_freq.to(position_ids.device)
        emb = torch.cat([freqs, freqs], dim=-1)
        return emb.cos(), emb.sin()

    def apply(self, q: torch.Tensor, k: torch.Tensor, position_ids: torch.Tensor):
        """Rotate q (B, Hq, S, D) and k (B, Hkv, S, D); angles position·inv_freq computed in-kernel in fp32."""
        if (q.shape[-1] % 16 == 0 and q.shape[-1] == self.dim and q.dtype == k.dtype
                and not needs_grad(q, k)):  # the fused kernel has no backward; apply_mrope has one
            qo = torch.empty_like(q, memory_format=torch.contiguous_format)
            ko = torch.empty_like(k, memory_format=torch.contiguous_format)
            pos = position_ids.to(device=q.device, dtype=torch.int32).contiguous()
            if pos.shape[1] == 1 and q.shape[0] > 1:
                pos = pos.expand(3, q.shape[0], pos.shape[2]).contiguous()
            # (B, H, S, D) tensors viewed as (B, S, H, D)
            qv, kv = q.transpose(1, 2), k.transpose(1, 2)
            qov, kov = qo.transpose(1, 2), ko.transpose(1, 2)
            qk_norm_rope(qv, kv, None, qov, kov, None, None, None, pos, self.inv_freq.to(q.device),
                         self.mrope_section, 0.0)
            return qo, ko
        cos_3d, sin_3d = self.compute_cos_sin(position_ids)
        return (apply_mrope(q, cos_3d, sin_3d, self.mrope_section),
                apply_mrope(k, cos_3d, sin_3d, self.mrope_section))

    def bind(self, position_ids: torch.Tensor) -> MRoPEBinding:
        """The `mrope_apply` callable for these positions (fusable by CudaFullAttention)."""
        return MRoPEBinding(self, position_ids)
