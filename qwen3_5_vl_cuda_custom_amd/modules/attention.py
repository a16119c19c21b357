"""CudaVisionAttention / CudaFullAttention (reference modules/attention.py:11-98)."""
from __future__ import annotations

import torch
from torch import nn

from ..kernels.backward import needs_grad
from ..kernels import (apply_rope, decode_attention, decode_attention_paged, flash_attention, flash_attention_cache,
                       flash_attention_cache_paged,
                       flash_attention_varlen, matmul_segments, qk_norm_rope, qk_norm_rope_attention,
                       qk_norm_rope_attention_ok, qk_norm_rope_paged, rmsnorm_matmul_segments)
from .kv_cache import PagedKVCache, StaticKVCache
from .linear import CudaLinear
from .norms import CudaRMSNorm, fused_norm_ok
from .rotary import MRoPEBinding


class CudaVisionAttention(nn.Module):
    """Non-causal vision attention with a fused `qkv` (3h, h) linear and `proj` (h, h), both with bias."""

    def __init__(self, hidden_size: int, num_heads: int) -> None:
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = hidden_size // num_heads
        self.scale = self.head_dim ** -0.5
        self.qkv = CudaLinear(hidden_size, 3 * hidden_size, bias=True)
        self.proj = CudaLinear(hidden_size, hidden_size, bias=True)

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                residual: torch.Tensor | None = None, *, cu_seqlens: torch.Tensor | None = None,
                max_seqlen: int | None = None) -> torch.Tensor:
        """x (B, S, h); cos/sin (S, D) (or (B|1, S, D)); images on the batch dim attend separately.

        cu_seqlens (int32, on the device) packs images of different sizes into
        one sequence (B = 1): image i is tokens [cu_seqlens[i], cu_seqlens[i+1])
        and attends only within itself (max_seqlen: the longest image).
        """
        B, S, h = x.shape
        H, D = self.num_heads, self.head_dim
        if needs_grad(x, residual, *self.parameters()):
            # training: the reference composition (modules/attention.py:34-42) on the differentiable ops
            if cu_seqlens is not None:
                raise NotImplementedError("CudaVisionAttention: packed images (cu_seqlens) have no backward; "
                                          "put the images on the batch dim to train")
            qkv = self.qkv(x).reshape(B, S, 3, H, D)
            q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
            q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
            o = flash_attention(q, k, v, scale=self.scale, is_causal=False, num_kv_groups=1)
            return self.proj(o.transpose(1, 2).reshape(B, S, h), residual=residual)
        qkv = self.qkv(x).view(B, S, 3, H, D)
        # q and k rotated by one launch: their 2H heads are one strided (B, 2H, S, D) view
        qk = apply_rope(qkv[:, :, :2].reshape(B, S, 2 * H, D).transpose(1, 2), cos, sin)
        q, k = qk[:, :H], qk[:, H:]
        v = qkv[:, :, 2].transpose(1, 2)
        o = torch.empty((B, S, H, D), dtype=x.dtype, device=x.device)
        if cu_seqlens is not None:
            if B != 1:
                raise ValueError("CudaVisionAttention: cu_seqlens packs the images into a batch of one")
            flash_attention_varlen(q[0], k[0], v[0], cu_seqlens, max_seqlen if max_seqlen is not None else S,
                                   self.scale, False, 1, out=o[0].transpose(0, 1))
        else:
            flash_attention(q, k, v, scale=self.scale, is_causal=False, num_kv_groups=1, out=o.transpose(1, 2))
        return self.proj(o.view(B, S, h), residual=residual)


class CudaFullAttention(nn.Module):
    """Causal GQA text attention with per-head q/k RMSNorm and mRoPE.

    Parameters (names and shapes as the reference): q_proj (Hq·D, h),
    k_proj/v_proj (Hkv·D, h), o_proj (h, Hq·D) (+ biases with attention_bias),
    q_norm/k_norm (D).

    forward(x, mrope_apply, past_kv=None) keeps the reference contract and
    returns (out, (k, v)) with k/v (B, Hkv, S_total, D). Additions:
      kv_cache=StaticKVCache  rotated k/v are written in place at each
                              sequence's length and attention runs over the
                              ragged cache: decode when S == 1, else a
                              prefill chunk whose token i attends causally to
                              the cache rows up to its own (lens[b] + i)
      kv_cache=PagedKVCache   the same over a paged cache: decode and prefill
                              chunks read the pages in place through the
                              block table; returns (k_pages, v_pages)
      residual=tensor         added to o_proj's output in the GEMM epilogue
      input_norm=CudaRMSNorm  x is the layer input before this RMSNorm; for
                              decode shapes (at most 32 tokens, bf16) the norm
                              runs inside the q/k/v projection, else first
    When `mrope_apply` is a TextMRoPE.bind(...) binding, q/k normalisation and
    rotation run as one fused kernel on the projection outputs; for a prefill
    without past_kv (bf16, GQA groups a multiple of 4), k's runs alone and q's
    inside the attention kernel (qk_norm_rope_attention).
    """

    def __init__(self, hidden_size: int, num_heads: int, num_kv_heads: int, head_dim: int | None = None,
                 rms_norm_eps: float = 1e-6, attention_bias: bool = False) -> None:
        super().__init__()
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.num_kv_groups = num_heads // num_kv_heads
        self.head_dim = head_dim or (hidden_size // num_heads)
        self.scale = self.head_dim ** -0.5
        self.q_proj = CudaLinear(hidden_size, num_heads * self.head_dim, bias=attention_bias)
        self.k_proj = CudaLinear(hidden_size, num_kv_heads * self.head_dim, bias=attention_bias)
        self.v_proj = CudaLinear(hidden_size, num_kv_heads * self.head_dim, bias=attention_bias)
        self.o_proj = CudaLinear(num_heads * self.head_dim, hidden_size, bias=attention_bias)
        self.q_norm = CudaRMSNorm(self.head_dim, eps=rms_norm_eps)
        self.k_norm = CudaRMSNorm(self.head_dim, eps=rms_norm_eps)

    def _fusable(self, mrope_apply, x: torch.Tensor) -> bool:
        return (isinstance(mrope_apply, MRoPEBinding) and mrope_apply.rope.dim == self.head_dim
                and self.head_dim % 16 == 0 and self.head_dim <= 256 and x.is_cuda)

    def forward(self, x: torch.Tensor, mrope_apply, past_kv: tuple[torch.Tensor, torch.Tensor] | None = None, *,
                kv_cache: StaticKVCache | PagedKVCache | None = None, residual: torch.Tensor | None = None,
                input_norm: CudaRMSNorm | None = None):
        B, S, _ = x.shape
        Hq, Hkv, D = self.num_heads, self.num_kv_heads, self.head_dim
        if needs_grad(x, residual, *self.parameters()):
            return self._forward_autograd(x, mrope_apply, past_kv, kv_cache, residual, input_norm)
        # q/k/v projections in one GEMM over the three weights (no concatenated
        # copy); q, k, v are column views of its output.
        weights = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight)
        biases = (self.q_proj.bias, self.k_proj.bias, self.v_proj.bias)
        if input_norm is not None and fused_norm_ok(x, input_norm):
            qkv = rmsnorm_matmul_segments(x, input_norm.weight, input_norm.eps, weights, biases)
        else:
            if input_norm is not None:
                x = input_norm(x)
            qkv = matmul_segments(x, weights, biases)
        q = qkv[..., :Hq * D].view(B, S, Hq, D)
        k = qkv[..., Hq * D:(Hq + Hkv) * D].view(B, S, Hkv, D)
        v = qkv[..., (Hq + Hkv) * D:].view(B, S, Hkv, D)
        o = torch.empty((B, S, Hq, D), dtype=x.dtype, device=x.device)

        if kv_cache is not None:
            if past_kv is not None:
                raise ValueError("pass either past_kv or kv_cache, not both")
            if not self._fusable(mrope_apply, x):
                raise ValueError("kv_cache decoding needs mrope_apply = TextMRoPE.bind(position_ids)")
            if kv_cache.batch != B:
                raise ValueError(f"kv_cache holds {kv_cache.batch} sequences, the input has {B}")
            rope = mrope_apply.rope
            pos = mrope_apply.positions_int32(x.device, B, S)
            if isinstance(kv_cache, PagedKVCache):
                kv_cache.check_kernels(self.num_kv_groups)
            kv_cache.reserve(S)  # raises, before any launch, if a sequence would overflow the cache
            if isinstance(kv_cache, PagedKVCache):
                return self._forward_paged(q, k, v, o, pos, rope, kv_cache, residual)
            kc, vc = kv_cache.k.transpose(1, 2), kv_cache.v.transpose(1, 2)  # (B, cap, Hkv, D) views
            # The new tokens' K/V rows go to cache rows [lens[b], lens[b] + S).
            qk_norm_rope(q, k, v, q, kc, vc, self.q_norm.weight, self.k_norm.weight, pos, rope.inv_freq,
                         rope.mrope_section, self.q_norm.eps, dst_seq_offset=kv_cache.lens,
                         dst_seq_cap=kv_cache.capacity)
            if S == 1:
                # attends to lens + 1 rows (the new token's included), then lens += 1
                decode_attention(q[:, 0], kv_cache.k, kv_cache.v, kv_cache.lens, self.scale, out=o[:, 0],
                                 max_len=kv_cache.capacity, append=True)
            else:
                # Prefill chunk: token i of sequence b sits at row lens[b] + i and
                # attends causally to rows [0, lens[b] + i]; then lens += S.
                flash_attention_cache(q.transpose(1, 2), kv_cache.k, kv_cache.v, kv_cache.lens, self.scale,
                                      self.num_kv_groups, out=o.transpose(1, 2), advance=True)
            return self.o_proj(o.view(B, S, Hq * D), residual=residual), (kv_cache.k, kv_cache.v)

        if self._fusable(mrope_apply, x):
            rope = mrope_apply.rope
            pos = mrope_apply.positions_int32(x.device, B, S)
            if (past_kv is None and self.q_norm.weight.dtype == q.dtype
                    and qk_norm_rope_attention_ok(q, k, self.num_kv_groups, v)):
                # k normalised and rotated in place; q inside the attention kernel
                qk_norm_rope_attention(q, k, v, self.q_norm.weight, self.k_norm.weight, pos, rope.inv_freq,
                                       rope.mrope_section, self.q_norm.eps, self.scale, True, out=o)
                return self.o_proj(o.view(B, S, Hq * D), residual=residual), (k.transpose(1, 2), v.transpose(1, 2))
            qk_norm_rope(q, k, None, q, k, None, self.q_norm.weight, self.k_norm.weight, pos, rope.inv_freq,
                         rope.mrope_section, self.q_norm.eps)
            qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        else:
            qh = self.q_norm(q).transpose(1, 2)
            kh = self.k_norm(k).transpose(1, 2)
            vh = v.transpose(1, 2)
            qh, kh = mrope_apply(qh, kh)
        if past_kv is not None:
            kh = torch.cat([past_kv[0], kh], dim=2)
            vh = torch.cat([past_kv[1], vh], dim=2)
        is_causal = qh.shape[2] == kh.shape[2]
        flash_attention(qh, kh, vh, scale=self.scale, is_causal=is_causal, num_kv_groups=self.num_kv_groups,
                        out=o.transpose(1, 2))
        return self.o_proj(o.view(B, S, Hq * D), residual=residual), (kh, vh)

    def _forward_autograd(self, x, mrope_apply, past_kv, kv_cache, residual, input_norm):
        """Training: the reference composition (modules/attention.py:75-98) on the differentiable ops
        (projections, q/k RMSNorm, mRoPE, attention and o_proj each with its own backward)."""
        if kv_cache is not None:
            raise NotImplementedError("CudaFullAttention: kv_cache decoding has no backward; run it under "
                                      "torch.no_grad() or torch.inference_mode()")
        B, S, _ = x.shape
        Hq, Hkv, D = self.num_heads, self.num_kv_heads, self.head_dim
        if input_norm is not None:
            x = input_norm(x)
        q = self.q_norm(self.q_proj(x).view(B, S, Hq, D)).transpose(1, 2)
        k = self.k_norm(self.k_proj(x).view(B, S, Hkv, D)).transpose(1, 2)
        v = self.v_proj(x).view(B, S, Hkv, D).transpose(1, 2)
        q, k = mrope_apply(q, k)
        if past_kv is not None:
            k = torch.cat([past_kv[0], k], dim=2)
            v = torch.cat([past_kv[1], v], dim=2)
        o = flash_attention(q, k, v, scale=self.scale, is_causal=q.shape[2] == k.shape[2],
                            num_kv_groups=self.num_kv_groups)
        return self.o_proj(o.transpose(1, 2).reshape(B, S, Hq * D), residual=residual), (k, v)

    def _forward_paged(self, q, k, v, o, pos, rope, kv_cache: PagedKVCache, residual):
        B, S, Hq, D = q.shape
        pt = kv_cache.block_table
        # The new tokens' K/V rows go to cache rows [lens[b], lens[b] + S) through the block table.
        qk_norm_rope_paged(q, k, v, q, kv_cache.k_pages, kv_cache.v_pages, self.q_norm.weight, self.k_norm.weight,
                           pos, rope.inv_freq, rope.mrope_section, self.q_norm.eps, pt, kv_cache.lens)
        if S == 1:
            decode_attention_paged(q[:, 0], kv_cache.k_pages, kv_cache.v_pages, pt, kv_cache.lens, self.scale,
                                   out=o[:, 0], append=True)
        else:
            # Prefill chunk: the ragged chunk kernel reads the pages in place through the block table.
            flash_attention_cache_paged(q.transpose(1, 2), kv_cache.k_pages, kv_cache.v_pages, pt, kv_cache.lens,
                                        self.scale, self.num_kv_groups, out=o.transpose(1, 2), advance=True)
        return self.o_proj(o.view(B, S, Hq * D), residual=residual), (kv_cache.k_pages, kv_cache.v_pages)
