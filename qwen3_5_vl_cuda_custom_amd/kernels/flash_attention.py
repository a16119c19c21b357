"""flash_attention (reference kernels/flash_attention.py:82-100) and ragged-cache decode attention."""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check, mfma_operand, note_slow_path
from .backward import FlashAttentionFunction, needs_grad


MFMA_HEAD_DIMS = (64, 72, 80, 96, 128)


def _attn_operands(op: str, D: int, o: torch.Tensor | None, *ts):
    """q/k/v as the MFMA attention kernels read them (aligned copies where needed);
    calls that only the SIMT kernel takes are reported."""
    out = [mfma_operand(op, t) for t in ts]
    if ts[0].dtype == torch.bfloat16:
        if D not in MFMA_HEAD_DIMS:
            note_slow_path(op, f"head_dim {D} (the MFMA kernels take {MFMA_HEAD_DIMS})")
        elif o is not None and (o.data_ptr() % 8 or any(o.stride(i) % 8 for i in range(o.dim() - 1))):
            note_slow_path(op, "the output view is not 8-byte aligned with strides in multiples of 8")
    return out


def _s4(t: torch.Tensor):
    return t.stride(0), t.stride(1), t.stride(2)


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, is_causal: bool = True,
                    num_kv_groups: int = 1, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(scale·QKᵀ [+ causal mask])·V with GQA.

    q (B, Hq, Sq, D), k/v (B, Hkv, Sk, D) with Hq = Hkv·num_kv_groups; query
    head h reads KV head h // num_kv_groups. Any strides are accepted as long as
    the head dim is contiguous (no copies). Causal masks key j > query i.
    `out`, when given, is a (B, Hq, Sq, D) view written in place.
    """
    if needs_grad(q, k, v):
        if out is not None:
            raise ValueError("flash_attention: out= is not supported when autograd records the op")
        return FlashAttentionFunction.apply(q, k, v, scale, is_causal, num_kv_groups)
    return _flash_fwd(q, k, v, scale, is_causal, num_kv_groups, out, None)


def flash_attention_lse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, is_causal: bool = True,
                        num_kv_groups: int = 1) -> tuple[torch.Tensor, torch.Tensor]:
    """flash_attention that also returns the row log-sum-exp of the scaled scores, lse (B, Hq, Sq) fp32
    (the forward schema's second output, csrc/flash_attention_op.cpp:14), which the backward reads."""
    B, Hq, Sq = q.shape[:3]
    lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=q.device)
    return _flash_fwd(q, k, v, scale, is_causal, num_kv_groups, None, lse), lse


def _flash_fwd(q, k, v, scale, is_causal, num_kv_groups, out, lse):
    check("flash_attention", q, k, v)
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    q, k, v = _attn_operands("flash_attention", q.shape[-1], out, q, k, v)
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    if k.shape != v.shape or k.shape[0] != B or k.shape[3] != D:
        raise ValueError(f"flash_attention: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if Hkv * num_kv_groups != Hq:
        raise ValueError(f"flash_attention: Hq={Hq} != Hkv={Hkv} * num_kv_groups={num_kv_groups}")
    o = out if out is not None else torch.empty((B, Hq, Sq, D), dtype=q.dtype, device=q.device)
    if o.shape != (B, Hq, Sq, D) or o.stride(-1) != 1:
        raise ValueError("flash_attention: out must be (B, Hq, Sq, D) with a contiguous head dim")
    _lib.call("q3_flash_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), _lib.ptr(lse), B, Hq, Hkv, Sq,
              Sk, D, _lib.i64s(*_s4(q), *_s4(k), *_s4(v), *_s4(o)), float(scale), int(bool(is_causal)),
              _lib.dtype_code(q.dtype), _lib.stream())
    return o


def qk_norm_rope_attention_ok(q: torch.Tensor, k: torch.Tensor, num_kv_groups: int,
                              v: torch.Tensor | None = None) -> bool:
    """Whether qk_norm_rope_attention covers these (B, S, H, D) views (else use
    qk_norm_rope followed by flash_attention). Mirrors every check of the C
    entry point (q3_qk_norm_rope_attention): bf16, D in (64, 128), GQA groups
    a multiple of 4, 16-byte aligned base pointers, batch / head / sequence
    strides that are multiples of 8 elements, a contiguous head dim, and 32-bit
    offsets within a KV head's rows ((S + 1) * seq stride * 2 < 2^31)."""
    B, S, _, D = q.shape
    ts = (q, k) if v is None else (q, k, v)
    if not (q.is_cuda and all(t.dtype == torch.bfloat16 for t in ts) and D in (64, 128)
            and num_kv_groups % 4 == 0 and S > 0 and B * S < 2 ** 31):
        return False
    for t in ts:
        if t.data_ptr() % 16 or t.stride(-1) != 1 or any(t.stride(i) % 8 for i in range(3)):
            return False
    return (S + 1) * k.stride(1) * 2 < 2 ** 31


def qk_norm_rope_attention(q_in: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_weight: torch.Tensor,
                           k_weight: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor, mrope_section,
                           eps: float, scale: float, is_causal: bool = True, *,
                           out: torch.Tensor | None = None) -> torch.Tensor:
    """q/k RMSNorm + mRoPE + attention of one prefill (reference modules/attention.py:83-96) in two launches.

    q_in (B, S, Hq, D), k/v (B, S, Hkv, D) views of the projection output (any
    strides, D contiguous); positions (3, B, S) int32, inv_freq (D/2) fp32 on
    the device. k is normalised and rotated in place; q is normalised and
    rotated inside the attention kernel as it is read (q_in is unchanged).
    Returns o (B, S, Hq, D) (or writes `out`, such a view). Equal to
    qk_norm_rope followed by flash_attention up to the summation order of each
    q row's sum of squares. bf16, D in (64, 128), GQA groups a multiple of 4.
    """
    check("qk_norm_rope_attention", q_in, k, v)
    B, S, Hq, D = q_in.shape
    Hkv = k.shape[2]
    if k.shape != v.shape or tuple(k.shape[:2]) != (B, S) or k.shape[3] != D or Hq % Hkv:
        raise ValueError(f"qk_norm_rope_attention: q {tuple(q_in.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if not qk_norm_rope_attention_ok(q_in, k, Hq // Hkv, v):
        raise ValueError("qk_norm_rope_attention: bf16, D in (64, 128), GQA groups a multiple of 4, 16-byte "
                         "aligned views with strides in multiples of 8 only")
    if (positions.dtype != torch.int32 or not positions.is_cuda or tuple(positions.shape) != (3, B, S)
            or not positions.is_contiguous()):
        raise ValueError(f"qk_norm_rope_attention: positions must be a contiguous int32 (3, {B}, {S}) device tensor")
    if inv_freq.dtype != torch.float32 or not inv_freq.is_cuda or inv_freq.numel() != D // 2:
        raise ValueError(f"qk_norm_rope_attention: inv_freq must be a float32 ({D // 2},) device tensor")
    for w in (q_weight, k_weight):
        if w.dtype != q_in.dtype or not w.is_cuda or w.shape != (D,) or not w.is_contiguous():
            raise ValueError(f"qk_norm_rope_attention: norm weights must be contiguous ({D},) device tensors")
    if sum(mrope_section) * 2 != D:
        raise ValueError(f"qk_norm_rope_attention: mrope_section {list(mrope_section)} must sum to D/2 = {D // 2}")
    if any(t.stride(-1) != 1 for t in (q_in, k, v)):
        raise ValueError("qk_norm_rope_attention: the head dim must be contiguous")
    o = out if out is not None else torch.empty((B, S, Hq, D), dtype=q_in.dtype, device=q_in.device)
    if o.shape != (B, S, Hq, D) or o.stride(-1) != 1:
        raise ValueError("qk_norm_rope_attention: out must be (B, S, Hq, D) with a contiguous head dim")
    ws, nws = _lib.workspace(_lib.lib().q3_qk_norm_rope_attention_workspace_bytes(B, S, D), q_in.device)
    qh, kh, vh, oh = (t.transpose(1, 2) for t in (q_in, k, v, o))  # (B, H, S, D) views
    _lib.call("q3_qk_norm_rope_attention", q_in.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
              q_weight.data_ptr(), k_weight.data_ptr(), positions.data_ptr(), inv_freq.data_ptr(), B, S, Hq, Hkv, D,
              _lib.i64s(*mrope_section), float(eps), _lib.i64s(*_s4(qh), *_s4(kh), *_s4(vh), *_s4(oh)),
              float(scale), int(bool(is_causal)), _lib.dtype_code(q_in.dtype), _lib.ptr(ws), nws, _lib.stream())
    return o


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, kv_lens: torch.Tensor,
                     scale: float, *, out: torch.Tensor | None = None, max_len: int | None = None,
                     append: bool = False, noalloc: bool = False) -> torch.Tensor:
    """One query token per sequence over a ragged KV cache (split-K flash decoding).

    q (B, Hq, D) (or (B, Hq, 1, D)); k_cache/v_cache (B, Hkv, cap, D); kv_lens
    (B,) int32 on the device — sequence b attends to cache rows [0, kv_lens[b]).
    `max_len` bounds every kv_lens[b] (default: cap). Returns (B, Hq, D).

    append=True is the decode step with the new token's row already at cache
    row kv_lens[b]: sequence b attends to kv_lens[b] + 1 rows and kv_lens is
    then incremented in place (stream-ordered, no host synchronisation).
    noalloc=True (with append=True, and `out` given) runs the step with the
    library's static per-GPU scratch instead of a workspace tensor: no
    allocation at all, for code that cannot allocate; calls overlapping in
    time on one GPU must not use it.
    """
    check("decode_attention", q, k_cache, v_cache)
    if q.dim() == 4:
        q = q[:, :, 0]
    B, Hq, D = q.shape
    Hkv, cap = k_cache.shape[1], k_cache.shape[2]
    if kv_lens.dtype != torch.int32 or not kv_lens.is_cuda or kv_lens.shape != (B,) or kv_lens.stride(0) != 1:
        raise ValueError("decode_attention: kv_lens must be a contiguous int32 (B,) device tensor")
    ml = int(max_len) if max_len is not None else cap
    strides = (q.stride(0), q.stride(1), *_s4(k_cache), *_s4(v_cache))
    if noalloc:
        if not append or out is None:
            raise ValueError("decode_attention: noalloc=True is the decode step (append=True) into a given `out`")
        _lib.call("q3_decode_attention_step_noalloc", q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                  kv_lens.data_ptr(), out.data_ptr(), B, Hq, Hkv, D, ml,
                  _lib.i64s(*strides, out.stride(0), out.stride(1)), float(scale), _lib.dtype_code(q.dtype),
                  _lib.stream())
        return out
    o = out if out is not None else torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    ws, nws = _lib.workspace(_lib.lib().q3_decode_attention_workspace_bytes(B, Hq, Hkv, ml, D), q.device)
    _lib.call("q3_decode_attention_step" if append else "q3_decode_attention", q.data_ptr(), k_cache.data_ptr(),
              v_cache.data_ptr(), kv_lens.data_ptr(),
              o.data_ptr(), B, Hq, Hkv, D, ml,
              _lib.i64s(q.stride(0), q.stride(1), *_s4(k_cache), *_s4(v_cache), o.stride(0), o.stride(1)),
              float(scale), _lib.dtype_code(q.dtype), _lib.ptr(ws), nws, _lib.stream())
    return o


def decode_attention_paged(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor, block_table: torch.Tensor,
                           kv_lens: torch.Tensor, scale: float, *, out: torch.Tensor | None = None,
                           append: bool = False, status: torch.Tensor | None = None) -> torch.Tensor:
    """decode_attention over a paged cache (no reference counterpart: the paged form of the decode loop's cache).

    q (B, Hq, D); k_pages/v_pages (num_pages, Hkv, page_rows, D) pools; block_table
    (B, max_pages) int32 on the device: cache row r of sequence b is row
    r % page_rows of page block_table[b, r // page_rows]. kv_lens (B,) int32.
    append=True: the step (the new token's row is already appended; attends to
    kv_lens[b] + 1 rows, then kv_lens += 1 in place). A page id outside the
    pool reads as zero rows and sets bit 1 of `status` (default: the device's
    status word, see _lib.device_status).
    """
    check("decode_attention_paged", q, k_pages, v_pages)
    if q.dim() == 4:
        q = q[:, :, 0]
    B, Hq, D = q.shape
    num_pages, Hkv, page_rows = k_pages.shape[0], k_pages.shape[1], k_pages.shape[2]
    if k_pages.shape != v_pages.shape or k_pages.shape[3] != D or k_pages.stride(-1) != 1 or v_pages.stride(-1) != 1:
        raise ValueError(f"decode_attention_paged: q {tuple(q.shape)}, pages {tuple(k_pages.shape)}")
    if (block_table.dtype != torch.int32 or not block_table.is_cuda or block_table.dim() != 2
            or block_table.shape[0] != B or not block_table.is_contiguous()):
        raise ValueError("decode_attention_paged: block_table must be a contiguous int32 (B, max_pages) device tensor")
    if kv_lens.dtype != torch.int32 or not kv_lens.is_cuda or kv_lens.shape != (B,) or kv_lens.stride(0) != 1:
        raise ValueError("decode_attention_paged: kv_lens must be a contiguous int32 (B,) device tensor")
    max_pages = block_table.shape[1]
    st = status if status is not None else _lib.status_word(q.device)
    o = out if out is not None else torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    ws, nws = _lib.workspace(_lib.lib().q3_decode_attention_workspace_bytes(B, Hq, Hkv, max_pages * page_rows, D),
                             q.device)
    _lib.call("q3_decode_attention_paged", q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(),
              block_table.data_ptr(), max_pages, page_rows, num_pages, kv_lens.data_ptr(), int(bool(append)),
              o.data_ptr(), B, Hq, Hkv, D,
              _lib.i64s(q.stride(0), q.stride(1), k_pages.stride(0), k_pages.stride(1), k_pages.stride(2),
                        v_pages.stride(0), v_pages.stride(1), v_pages.stride(2), o.stride(0), o.stride(1)),
              float(scale), _lib.dtype_code(q.dtype), _lib.ptr(ws), nws, st.data_ptr(), _lib.stream())
    return o


def flash_attention_cache(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, kv_lens: torch.Tensor,
                          scale: float, num_kv_groups: int = 1, *, out: torch.Tensor | None = None,
                          advance: bool = False) -> torch.Tensor:
    """Causal attention of a prefill chunk over a ragged KV cache.

    q (B, Hq, Sq, D); k_cache/v_cache (B, Hkv, cap, D) whose rows
    [kv_lens[b], kv_lens[b] + Sq) already hold the chunk's keys/values;
    kv_lens (B,) int32 on the device. Query i of sequence b is the token at
    position kv_lens[b] + i and attends to cache rows [0, kv_lens[b] + i]
    (the causal mask of the whole sequence, bottom-right aligned for the
    chunk). advance=True adds Sq to kv_lens afterwards, in stream order.
    Returns (B, Hq, Sq, D).
    """
    check("flash_attention_cache", q, k_cache, v_cache)
    if q.stride(-1) != 1:
        q = q.contiguous()
    (q,) = _attn_operands("flash_attention_cache", q.shape[-1], out, q)
    if q.dtype == torch.bfloat16 and any(t.data_ptr() % 16 or any(t.stride(i) % 8 for i in range(3))
                                         for t in (k_cache, v_cache)):
        note_slow_path("flash_attention_cache", "the caches are not 16-byte aligned with strides in multiples of 8")
    B, Hq, Sq, D = q.shape
    Hkv, cap = k_cache.shape[1], k_cache.shape[2]
    if k_cache.shape != v_cache.shape or k_cache.shape[0] != B or k_cache.shape[3] != D:
        raise ValueError(f"flash_attention_cache: q {tuple(q.shape)}, caches {tuple(k_cache.shape)}")
    if k_cache.stride(-1) != 1 or v_cache.stride(-1) != 1:
        raise ValueError("flash_attention_cache: the caches' head dim must be contiguous")
    if Hkv * num_kv_groups != Hq:
        raise ValueError(f"flash_attention_cache: Hq={Hq} != Hkv={Hkv} * num_kv_groups={num_kv_groups}")
    if kv_lens.dtype != torch.int32 or not kv_lens.is_cuda or kv_lens.shape != (B,) or kv_lens.stride(0) != 1:
        raise ValueError("flash_attention_cache: kv_lens must be a contiguous int32 (B,) device tensor")
    o = out if out is not None else torch.empty((B, Hq, Sq, D), dtype=q.dtype, device=q.device)
    if o.shape != (B, Hq, Sq, D) or o.stride(-1) != 1:
        raise ValueError("flash_attention_cache: out must be (B, Hq, Sq, D) with a contiguous head dim")
    _lib.call("q3_flash_attention_cache", q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), kv_lens.data_ptr(),
              o.data_ptr(), B, Hq, Hkv, Sq, cap, D, _lib.i64s(*_s4(q), *_s4(k_cache), *_s4(v_cache), *_s4(o)),
              float(scale), int(bool(advance)), _lib.dtype_code(q.dtype), _lib.stream())
    return o



def flash_attention_cache_paged(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                                block_table: torch.Tensor, kv_lens: torch.Tensor, scale: float,
                                num_kv_groups: int = 1, *, out: torch.Tensor | None = None, advance: bool = False,
                                status: torch.Tensor | None = None) -> torch.Tensor:
    """flash_attention_cache over a paged cache, read in place through the block table (no copy).

    q (B, Hq, Sq, D); k_pages/v_pages (num_pages, Hkv, page_rows, D) pools;
    block_table (B, max_pages) int32 on the device (cache row r of sequence b is
    row r % page_rows of page block_table[b, r // page_rows]); the chunk's rows
    [kv_lens[b], kv_lens[b] + Sq) already hold its keys/values. Query i of
    sequence b attends causally to cache rows [0, kv_lens[b] + i]; advance=True
    adds Sq to kv_lens afterwards. Same kernel and arithmetic as
    flash_attention_cache, so a paged call returns the contiguous call's output
    bit for bit. bf16, D = 128, at most 512 pages a
    sequence. A page id outside the pool reads as zero rows and sets bit 1 of
    `status` (default: the device's status word).
    """
    check("flash_attention_cache_paged", q, k_pages, v_pages)
    if q.stride(-1) != 1:
        q = q.contiguous()
    (q,) = _attn_operands("flash_attention_cache_paged", q.shape[-1], out, q)
    B, Hq, Sq, D = q.shape
    num_pages, Hkv, page_rows = k_pages.shape[0], k_pages.shape[1], k_pages.shape[2]
    if k_pages.shape != v_pages.shape or k_pages.shape[3] != D or k_pages.stride(-1) != 1 or v_pages.stride(-1) != 1:
        raise ValueError(f"flash_attention_cache_paged: q {tuple(q.shape)}, pages {tuple(k_pages.shape)}")
    if Hkv * num_kv_groups != Hq:
        raise ValueError(f"flash_attention_cache_paged: Hq={Hq} != Hkv={Hkv} * num_kv_groups={num_kv_groups}")
    if (block_table.dtype != torch.int32 or not block_table.is_cuda or block_table.dim() != 2
            or block_table.shape[0] != B or not block_table.is_contiguous()):
        raise ValueError("flash_attention_cache_paged: block_table must be a contiguous int32 (B, max_pages) "
                         "device tensor")
    if kv_lens.dtype != torch.int32 or not kv_lens.is_cuda or kv_lens.shape != (B,) or kv_lens.stride(0) != 1:
        raise ValueError("flash_attention_cache_paged: kv_lens must be a contiguous int32 (B,) device tensor")
    o = out if out is not None else torch.empty((B, Hq, Sq, D), dtype=q.dtype, device=q.device)
    if o.shape != (B, Hq, Sq, D) or o.stride(-1) != 1:
        raise ValueError("flash_attention_cache_paged: out must be (B, Hq, Sq, D) with a contiguous head dim")
    st = status if status is not None else _lib.status_word(q.device)
    _lib.call("q3_flash_attention_cache_paged", q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(),
              block_table.data_ptr(), block_table.shape[1], page_rows, num_pages, kv_lens.data_ptr(), o.data_ptr(),
              B, Hq, Hkv, Sq, D,
              _lib.i64s(*_s4(q), *_s4(k_pages), *_s4(v_pages), *_s4(o)), float(scale), int(bool(advance)),
              _lib.dtype_code(q.dtype), st.data_ptr(), _lib.stream())
    return o

def flash_attention_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
                           max_seqlen: int, scale: float, is_causal: bool = False, num_kv_groups: int = 1, *,
                           out: torch.Tensor | None = None) -> torch.Tensor:
    """Attention over packed variable-length sequences (HF's cu_seqlens form).

    q (Hq, total, D), k/v (Hkv, total, D), any strides with D contiguous;
    cu_seqlens (n+1,) int32 on the device with cu_seqlens[0] = 0 and
    cu_seqlens[-1] = total: sequence b is rows [cu[b], cu[b+1]) and attends only
    within itself (causally when is_causal). max_seqlen bounds every length.
    Returns (Hq, total, D) (`out`, when given, is written in place).
    """
    check("flash_attention_varlen", q, k, v)
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    q, k, v = _attn_operands("flash_attention_varlen", q.shape[-1], out, q, k, v)
    Hq, total, D = q.shape
    Hkv = k.shape[0]
    if k.shape != v.shape or k.shape[1] != total or k.shape[2] != D or Hkv * num_kv_groups != Hq:
        raise ValueError(f"flash_attention_varlen: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if cu_seqlens.dtype != torch.int32 or not cu_seqlens.is_cuda or cu_seqlens.dim() != 1:
        raise ValueError("flash_attention_varlen: cu_seqlens must be a 1-D int32 device tensor")
    o = out if out is not None else torch.empty((Hq, total, D), dtype=q.dtype, device=q.device)
    if o.shape != (Hq, total, D) or o.stride(-1) != 1:
        raise ValueError("flash_attention_varlen: out must be (Hq, total, D) with a contiguous head dim")
    st = [q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1), o.stride(0), o.stride(1)]
    _lib.call("q3_flash_attention_varlen", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
              cu_seqlens.contiguous().data_ptr(), cu_seqlens.numel() - 1, total, int(max_seqlen), Hq, Hkv, D,
              _lib.i64s(*st), float(scale), int(bool(is_causal)), _lib.dtype_code(q.dtype), _lib.stream())
    return o
