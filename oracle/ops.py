"""Op-level CPU oracle: the reference's PyTorch fallbacks restated in float32.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Citations are relative to
the reference root `CUDA_qwen3_5-main/CUDA_qwen3_5-main/cuda_qwen3_vl/`.

All functions take CPU tensors and compute in the dtype they are given; the
tests call them with float32 tensors (bf16-rounded inputs upcast to fp32).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = [
    "linear", "batched_gemm", "conv3d_patch", "flash_attention", "decode_attention", "chunk_attention",
    "interleave_cos_sin", "rotate_half_apply", "mrope_inv_freq", "mrope_cos_sin",
    "apply_mrope", "apply_rope", "rmsnorm", "layernorm", "swiglu", "residual_add",
    "gelu_tanh", "softmax", "topk", "index_add", "round_bf16", "sigmoid_mul", "cross_entropy",
]


def round_bf16(t: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (round-to-nearest-even) and return float32: one op-boundary rounding."""
    return t.to(torch.bfloat16).to(torch.float32)


# ---------------------------------------------------------------- GEMMs

def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """Y = X·Wᵀ + b (nn.Linear layout). kernels/matmul.py:62-64 (`F.linear`)."""
    return F.linear(x, weight, bias)


def batched_gemm(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Y[e] = X[e]·W[e]ᵀ; x (E,M,K), w (E,N,K). kernels/moe_routing.py:173-176 (einsum)."""
    return torch.einsum("emk,enk->emn", x, w)


def conv3d_patch(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """Non-overlapping conv3d (stride == kernel) flattened to (N, E).

    kernels/conv3d_patch.py:13-14 and :26-29.
    """
    kernel_size = weight.shape[2:]
    return F.conv3d(x, weight, bias=bias, stride=kernel_size).reshape(x.shape[0], -1)


# ---------------------------------------------------------------- attention

def flash_attention(q, k, v, scale: float, is_causal: bool = True, num_kv_groups: int = 1):
    """softmax(scale·QKᵀ + causal)·V with GQA by KV expansion.

    kernels/flash_attention.py:13-18: KV head j serves query heads
    j*groups .. j*groups+groups-1 (expand on a new dim 2, then reshape), then
    `F.scaled_dot_product_attention(is_causal=..., scale=...)`. The causal mask is
    top-left aligned (query i sees keys 0..i), as SDPA defines it.
    """
    if num_kv_groups > 1:
        B, nkv, S, D = k.shape
        k = k[:, :, None].expand(B, nkv, num_kv_groups, S, D).reshape(B, nkv * num_kv_groups, S, D)
        v = v[:, :, None].expand(B, nkv, num_kv_groups, S, D).reshape(B, nkv * num_kv_groups, S, D)
    return F.scaled_dot_product_attention(q, k, v, is_causal=is_causal, scale=scale)


def decode_attention(q, k_cache, v_cache, kv_lens, scale: float, num_kv_groups: int):
    """One new query token per sequence over a ragged per-sequence KV cache.

    The reference decode step is `flash_attention` with Sq=1 and is_causal=False
    over the concatenated cache (modules/attention.py:89-96). With per-sequence
    lengths, sequence b attends to cache[b, :, :kv_lens[b]] only; this runs the
    reference attention on that slice, one sequence at a time.
    q (B,Hq,1,D); k_cache/v_cache (B,Hkv,cap,D); kv_lens (B,) int.
    """
    outs = []
    for b in range(q.shape[0]):
        L = int(kv_lens[b])
        outs.append(flash_attention(q[b:b + 1], k_cache[b:b + 1, :, :L], v_cache[b:b + 1, :, :L],
                                    scale, False, num_kv_groups))
    return torch.cat(outs, dim=0)


def chunk_attention(q, k_cache, v_cache, kv_lens, scale: float, num_kv_groups: int):
    """Causal attention of a prefill chunk over a ragged per-sequence KV cache.

    The chunk's Sq tokens of sequence b sit at cache rows kv_lens[b] + i; query
    i attends to rows [0, kv_lens[b] + i] of that sequence, i.e. the causal mask
    of the whole sequence restricted to the chunk's rows. The reference has no
    such form: its cache concat runs a chunk non-causally (is_causal = Sq == Sk,
    modules/attention.py:89-96). This is the attention of
    `flash_attention(..., is_causal=True)` (kernels/flash_attention.py:13-18,
    SDPA) over the whole sequence, kept for the chunk's rows, computed with an
    explicit boolean mask per sequence.
    q (B,Hq,Sq,D); k_cache/v_cache (B,Hkv,cap,D); kv_lens (B,) int.
    """
    B, Hq, Sq, D = q.shape
    outs = []
    for b in range(B):
        L = int(kv_lens[b])
        k = k_cache[b:b + 1, :, :L + Sq]
        v = v_cache[b:b + 1, :, :L + Sq]
        if num_kv_groups > 1:
            nkv = k.shape[1]
            k = k[:, :, None].expand(1, nkv, num_kv_groups, L + Sq, D).reshape(1, Hq, L + Sq, D)
            v = v[:, :, None].expand(1, nkv, num_kv_groups, L + Sq, D).reshape(1, Hq, L + Sq, D)
        keep = torch.arange(L + Sq)[None, :] <= (L + torch.arange(Sq))[:, None]
        outs.append(F.scaled_dot_product_attention(q[b:b + 1], k, v, attn_mask=keep.to(q.device), scale=scale))
    return torch.cat(outs, dim=0)


# ---------------------------------------------------------------- rotary

def interleave_cos_sin(cos_3d, sin_3d, mrope_section):
    """(3,B,S,D) cos/sin → (B,S,D) with the reference's chunked section layout.

    kernels/mrope.py:19-35: `mrope_section*2` is walked left to right; slice i
    takes columns [offset, offset+m) from axis i % 3.
    """
    sections = list(mrope_section) * 2
    cos_parts, sin_parts = [], []
    offset = 0
    for i, m in enumerate(sections):
        axis = i % 3
        cos_parts.append(cos_3d[axis, ..., offset:offset + m])
        sin_parts.append(sin_3d[axis, ..., offset:offset + m])
        offset += m
    return torch.cat(cos_parts, dim=-1), torch.cat(sin_parts, dim=-1)


def rotate_half_apply(x, cos, sin):
    """Rotate-half RoPE on the first D_rope = cos.shape[-1] dims; the tail passes through.

    kernels/mrope.py:38-50 (cos (B,S,D_rope) broadcast over heads) and
    kernels/rope.py:12-28 (also accepts cos (S,D_rope)). Only the first half of
    cos/sin is read: out1 = x1·c1 − x2·s1, out2 = x2·c1 + x1·s1.
    """
    D_rope = cos.shape[-1]
    half = D_rope // 2
    x_rot, x_pass = x[..., :D_rope], x[..., D_rope:]
    x1, x2 = x_rot[..., :half], x_rot[..., half:]
    if cos.dim() == 3:
        c, s = cos.unsqueeze(1), sin.unsqueeze(1)
    else:
        c, s = cos[None, None], sin[None, None]
    c1, s1 = c[..., :half], s[..., :half]
    rot = torch.cat([x1 * c1 - x2 * s1, x2 * c1 + x1 * s1], dim=-1)
    return torch.cat([rot, x_pass], dim=-1)


def mrope_inv_freq(dim: int, theta: float) -> torch.Tensor:
    """inv_freq = 1/theta^(arange(0,dim,2)/dim) in fp32. modules/rotary.py:43."""
    return 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))


def mrope_cos_sin(position_ids: torch.Tensor, dim: int, theta: float):
    """TextMRoPE.compute_cos_sin: position_ids (3,B,S) → cos/sin (3,B,S,dim) fp32.

    modules/rotary.py:46-55: freqs = pos·inv_freq, emb = cat(freqs, freqs).
    """
    inv_freq = mrope_inv_freq(dim, theta).to(position_ids.device)
    freqs = position_ids.float().unsqueeze(-1) * inv_freq
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def apply_mrope(x, cos_3d, sin_3d, mrope_section):
    """kernels/mrope.py:80-104: interleave, cast cos/sin to x dtype, rotate-half."""
    cos, sin = interleave_cos_sin(cos_3d, sin_3d, mrope_section)
    return rotate_half_apply(x, cos.to(x.dtype), sin.to(x.dtype))


def apply_rope(x, cos, sin):
    """kernels/rope.py:58-72: cast cos/sin to x dtype, rotate-half."""
    return rotate_half_apply(x, cos.to(x.dtype), sin.to(x.dtype))


# ---------------------------------------------------------------- norms / elementwise

def rmsnorm(x, weight, eps: float = 1e-6):
    """fp32 x·rsqrt(mean(x²)+eps)·w, cast back once. kernels/rmsnorm.py:12-17."""
    dtype = x.dtype
    x_fp = x.float()
    var = x_fp.pow(2).mean(dim=-1, keepdim=True)
    return (x_fp * torch.rsqrt(var + eps) * weight.float()).to(dtype)


def layernorm(x, weight, bias=None, eps: float = 1e-6):
    """F.layer_norm over the last dim. kernels/layernorm.py:13-14."""
    return F.layer_norm(x, (x.shape[-1],), weight, bias, eps)


def swiglu(gate, up):
    """silu(gate)·up. kernels/swiglu.py:13-14."""
    return F.silu(gate) * up


def residual_add(a, b):
    """a + b. kernels/residual_add.py:30."""
    return a + b


def gelu_tanh(x):
    """0.5x(1+tanh(√(2/π)(x+0.044715x³))). kernels/gelu_tanh.py:13-14."""
    return F.gelu(x, approximate="tanh")


def softmax(x):
    """Row softmax over the last dim. kernels/softmax.py:42."""
    return torch.softmax(x, dim=-1)


# ---------------------------------------------------------------- MoE routing

def topk(x, k: int):
    """Top-k values and int64 indices per row, ties broken by the lowest index.

    kernels/moe_routing.py:58-61 calls torch.topk; the CUDA kernel
    (csrc/moe_routing_op.cu:11-63) takes k rounds of a strict-`>` arg-max, so the
    lowest index wins among equal values. A stable descending sort has exactly
    that order.
    """
    vals, idx = torch.sort(x, dim=-1, descending=True, stable=True)
    return vals[..., :k].contiguous(), idx[..., :k].contiguous()


def index_add(target, source, index):
    """target[index[i]] += source[i] (in place, returns target). kernels/moe_routing.py:111-115."""
    target.index_add_(0, index, source)
    return target


# ---------------------------------------------------------------- the rest of the op namespace

def sigmoid_mul(x, gate):
    """x·sigmoid(gate). kernels/sigmoid_mul.py:12-13."""
    return x * torch.sigmoid(gate)


def cross_entropy(logits, targets, ignore_index: int = -100):
    """Mean over targets != ignore_index of logsumexp(row) − row[target].

    kernels/cross_entropy.py:56-64 (the op's path): per-token losses
    (csrc/cross_entropy_op.cu:10-62, 0 for an ignored target) summed and divided
    by the valid count clamped to at least 1, so a batch with every target
    ignored gives 0 where the fallback `F.cross_entropy` (:13-14) gives nan; the
    two agree otherwise. Differentiable in logits.
    """
    valid = targets != ignore_index
    safe = torch.where(valid, targets, torch.zeros_like(targets))
    lse = torch.logsumexp(logits, dim=-1)
    per_token = torch.where(valid, lse - logits.gather(-1, safe[:, None])[:, 0], torch.zeros_like(lse))
    return per_token.sum() / valid.sum().clamp(min=1)
