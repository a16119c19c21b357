"""Module-level CPU oracle: the reference's nn.Module compositions restated.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Parameters are passed as a
dict keyed by the reference's state_dict names (e.g. "self_attn.q_proj.weight"),
so a test can hand over `module.state_dict()` converted to CPU float32.

`rd` is applied to every op output. With `rd=identity` this is the float32
reference the bf16 GPU path is measured against; with `rd=ops.round_bf16` it
reproduces the reference's bf16 path, where every op rounds its output to bf16
(used where a discrete decision, the MoE routing, must see bf16 logits).
"""
from __future__ import annotations

import torch

from . import ops


def _ident(t):
    return t


def _get(p, prefix, name):
    return p.get(f"{prefix}{name}")


# ---------------------------------------------------------------- text

def full_attention(x, p, *, num_heads, num_kv_heads, head_dim, eps, cos_3d, sin_3d, mrope_section,
                   past_kv=None, prefix="", rd=_ident):
    """CudaFullAttention.forward, modules/attention.py:75-98.

    proj → (B,S,H,D) → q_norm/k_norm over D → (B,H,S,D) → mRoPE (the
    `mrope_apply` lambda of models/dense.py:68 → modules/rotary.py:57-59) →
    optional cache concat → attention (causal iff Sq == Sk) → (B,S,H·D) → o_proj.
    Returns (out, (k, v)).
    """
    B, S, _ = x.shape
    q = rd(ops.linear(x, p[prefix + "q_proj.weight"], _get(p, prefix, "q_proj.bias"))).reshape(B, S, num_heads, head_dim)
    k = rd(ops.linear(x, p[prefix + "k_proj.weight"], _get(p, prefix, "k_proj.bias"))).reshape(B, S, num_kv_heads, head_dim)
    v = rd(ops.linear(x, p[prefix + "v_proj.weight"], _get(p, prefix, "v_proj.bias"))).reshape(B, S, num_kv_heads, head_dim)
    q = rd(ops.rmsnorm(q, p[prefix + "q_norm.weight"], eps)).transpose(1, 2)
    k = rd(ops.rmsnorm(k, p[prefix + "k_norm.weight"], eps)).transpose(1, 2)
    v = v.transpose(1, 2)
    # The reference casts the fp32 cos/sin tables to the activation dtype before
    # its rotation kernel (kernels/mrope.py:92-93), so its bf16 path rotates with
    # bf16-rounded tables.
    cos_r, sin_r = rd(cos_3d), rd(sin_3d)
    q = rd(ops.apply_mrope(q, cos_r, sin_r, mrope_section))
    k = rd(ops.apply_mrope(k, cos_r, sin_r, mrope_section))
    if past_kv is not None:
        k = torch.cat([past_kv[0], k], dim=2)
        v = torch.cat([past_kv[1], v], dim=2)
    is_causal = q.shape[2] == k.shape[2]
    out = rd(ops.flash_attention(q, k, v, head_dim ** -0.5, is_causal, num_heads // num_kv_heads))
    out = out.transpose(1, 2).reshape(B, S, -1)
    return rd(ops.linear(out, p[prefix + "o_proj.weight"], _get(p, prefix, "o_proj.bias"))), (k, v)


def swiglu_mlp(x, p, prefix="", rd=_ident):
    """CudaSwiGLUMLP.forward, modules/mlp.py:19-22: down(swiglu(gate(x), up(x)))."""
    gate = rd(ops.linear(x, p[prefix + "gate_proj.weight"], _get(p, prefix, "gate_proj.bias")))
    up = rd(ops.linear(x, p[prefix + "up_proj.weight"], _get(p, prefix, "up_proj.bias")))
    act = rd(ops.swiglu(gate, up))
    return rd(ops.linear(act, p[prefix + "down_proj.weight"], _get(p, prefix, "down_proj.bias")))


def sparse_moe(x, p, *, top_k, norm_topk_prob=True, prefix="", rd=_ident, router_logits=None):
    """CudaSparseMoE.forward, modules/moe.py:54-85.

    logits = x·gate_weightᵀ (rounded to x dtype) → fp32 softmax → top-k
    (lowest index wins ties) → renormalise → cast to x dtype; then, for each
    expert e in ascending order, its (token, slot) pairs in ascending token
    order (`nonzero`), gate_up GEMM, swiglu on the two column halves, down GEMM,
    times the routing weight (in x dtype), index_add into the running output.
    `router_logits`, when given, replaces the router GEMM output (so a test can
    route with exactly the logits the device produced). Returns (out, logits).
    """
    B, S, H = x.shape
    x_flat = x.reshape(-1, H)
    gate_w = p[prefix + "gate_weight"]
    gate_up = p[prefix + "gate_up_proj"]
    down = p[prefix + "down_proj"]
    I = down.shape[2]
    if router_logits is None:
        router_logits = rd(ops.linear(x_flat, gate_w))
    probs = ops.softmax(router_logits.float())
    top_vals, top_idx = ops.topk(probs, top_k)
    if norm_topk_prob:
        top_vals = top_vals / top_vals.sum(dim=-1, keepdim=True)
    top_vals = rd(top_vals)
    final = torch.zeros_like(x_flat)
    for e in range(gate_w.shape[0]):
        mask = top_idx == e
        if not mask.any():
            continue
        token_idx, slot_idx = mask.nonzero(as_tuple=True)
        gu = rd(ops.linear(x_flat[token_idx], gate_up[e]))
        act = rd(ops.swiglu(gu[:, :I], gu[:, I:]))
        eo = rd(ops.linear(act, down[e]))
        weighted = rd(eo * top_vals[token_idx, slot_idx, None])
        final = rd(ops.index_add(final, weighted, token_idx))
    return final.reshape(B, S, H), router_logits


def text_decoder_layer(x, p, *, num_heads, num_kv_heads, head_dim, eps, cos_3d, sin_3d, mrope_section,
                       use_moe=False, top_k=0, past_kv=None, rd=_ident, router_logits=None):
    """CudaTextDecoderLayer.forward, modules/text_decoder.py:51-65.

    h = x + Attn(RMSNorm(x)); y = h + MLP(RMSNorm(h)). Returns (y, router_logits|None, (k,v)).
    """
    hn = rd(ops.rmsnorm(x, p["input_layernorm.weight"], eps))
    attn_out, new_kv = full_attention(hn, p, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                                      eps=eps, cos_3d=cos_3d, sin_3d=sin_3d, mrope_section=mrope_section,
                                      past_kv=past_kv, prefix="self_attn.", rd=rd)
    h = rd(ops.residual_add(attn_out, x))
    mlp_in = rd(ops.rmsnorm(h, p["post_attention_layernorm.weight"], eps))
    if use_moe:
        mlp_out, logits = sparse_moe(mlp_in, p, top_k=top_k, prefix="mlp.", rd=rd, router_logits=router_logits)
    else:
        mlp_out, logits = swiglu_mlp(mlp_in, p, prefix="mlp.", rd=rd), None
    return rd(ops.residual_add(mlp_out, h)), logits, new_kv


# ---------------------------------------------------------------- vision

def vision_attention(x, p, *, num_heads, cos, sin, prefix="", rd=_ident):
    """CudaVisionAttention.forward, modules/attention.py:25-42 (non-causal, groups 1)."""
    B, S, h = x.shape
    hd = h // num_heads
    qkv = rd(ops.linear(x, p[prefix + "qkv.weight"], p[prefix + "qkv.bias"])).reshape(B, S, 3, num_heads, hd)
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    # cos/sin cast to the activation dtype first, as kernels/rope.py:60-61 does.
    q = rd(ops.apply_rope(q, rd(cos), rd(sin)))
    k = rd(ops.apply_rope(k, rd(cos), rd(sin)))
    out = rd(ops.flash_attention(q, k, v, hd ** -0.5, False, 1)).transpose(1, 2).reshape(B, S, -1)
    return rd(ops.linear(out, p[prefix + "proj.weight"], p[prefix + "proj.bias"]))


def vision_mlp(x, p, prefix="", rd=_ident):
    """CudaVisionMLP.forward, modules/mlp.py:33-34: fc2(gelu_tanh(fc1(x)))."""
    h = rd(ops.linear(x, p[prefix + "linear_fc1.weight"], p[prefix + "linear_fc1.bias"]))
    h = rd(ops.gelu_tanh(h))
    return rd(ops.linear(h, p[prefix + "linear_fc2.weight"], p[prefix + "linear_fc2.bias"]))


def vision_block(x, p, *, num_heads, cos, sin, eps=1e-6, rd=_ident):
    """CudaVisionBlock.forward, modules/vision_block.py:21-24."""
    a = vision_attention(rd(ops.layernorm(x, p["norm1.weight"], p["norm1.bias"], eps)), p,
                         num_heads=num_heads, cos=cos, sin=sin, prefix="attn.", rd=rd)
    x = rd(ops.residual_add(a, x))
    m = vision_mlp(rd(ops.layernorm(x, p["norm2.weight"], p["norm2.bias"], eps)), p, prefix="mlp.", rd=rd)
    return rd(ops.residual_add(m, x))


def patch_embed(x, weight, bias, in_channels, temporal_patch_size, patch_size):
    """CudaVisionPatchEmbed.forward, modules/vision_patch.py:35-39: (N, C·T·P·P) → conv3d_patch."""
    if x.dim() == 2:
        x = x.view(-1, in_channels, temporal_patch_size, patch_size, patch_size)
    return ops.conv3d_patch(x, weight, bias)


def vision_rope_tables(grid_thw, head_dim: int, theta: float = 10000.0, merge: int = 2):
    """2D-rope cos/sin (total_tokens, head_dim) for a list of (t, h, w) grids, in fp32.

    models/common.py:44-54 (inv_freq over rotary_dim = head_dim//2),
    :80-83 (freq table = outer(arange(max_hw), inv_freq)), :85-120 (merge-block
    (row, col) coordinates, repeated t times) and :192-195 (emb = cat(rot, rot)).
    The reference rounds emb to the activation dtype before cos/sin
    (:193); this restatement keeps fp32, as HF does.
    """
    rotary_dim = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))
    max_hw = max(max(h, w) for _, h, w in grid_thw)
    table = torch.outer(torch.arange(max_hw, dtype=torch.float32), inv_freq)
    coords = []
    for t, h, w in grid_thw:
        mh, mw = h // merge, w // merge
        br = torch.arange(mh)[:, None, None, None] * merge + torch.arange(merge)[None, None, :, None]
        bc = torch.arange(mw)[None, :, None, None] * merge + torch.arange(merge)[None, None, None, :]
        r = br.expand(mh, mw, merge, merge).reshape(-1)
        c = bc.expand(mh, mw, merge, merge).reshape(-1)
        xy = torch.stack((r, c), dim=-1)
        coords.append(xy.repeat(t, 1) if t > 1 else xy)
    pos = torch.cat(coords, dim=0)
    rot = table[pos].flatten(1)
    emb = torch.cat((rot, rot), dim=-1)
    return emb.cos(), emb.sin()


def patch_merger(x, p, *, merge: int, postshuffle: bool, prefix: str = "", eps: float = 1e-6, rd=_ident):
    """CudaVisionPatchMerger.forward, modules/vision_patch.py:58-68: LayerNorm (over the patch
    hidden, or over merge^2 patches when postshuffle), rows of merge^2 tokens, fc1, gelu_tanh, fc2."""
    mh = x.shape[-1] * merge * merge if not postshuffle else p[prefix + "norm.weight"].shape[0]
    if postshuffle:
        x = rd(ops.layernorm(x.reshape(-1, mh), p[prefix + "norm.weight"], p[prefix + "norm.bias"], eps))
    else:
        x = rd(ops.layernorm(x, p[prefix + "norm.weight"], p[prefix + "norm.bias"], eps)).reshape(-1, mh)
    h = rd(ops.gelu_tanh(rd(ops.linear(x, p[prefix + "linear_fc1.weight"], p[prefix + "linear_fc1.bias"]))))
    return rd(ops.linear(h, p[prefix + "linear_fc2.weight"], p[prefix + "linear_fc2.bias"]))


def pos_embed_interpolate(table, grid_thw, merge: int):
    """CudaVisionTower._fast_pos_embed_interpolate, models/common.py:122-174, in fp32.

    Per image: coordinates linspace(0, G-1, h) x linspace(0, G-1, w) on the
    G x G learned grid, bilinear weights over floor / clipped floor+1, the
    weighted sum of the four table rows, repeated over the t frames and
    permuted to the merge-block token order. Returns (total, hidden).
    """
    G = int(round(table.shape[0] ** 0.5))
    out = []
    for t, h, w in grid_thw:
        hi = torch.linspace(0, G - 1, h)
        wi = torch.linspace(0, G - 1, w)
        hf, wf = hi.int(), wi.int()
        hc, wc = (hf + 1).clip(max=G - 1), (wf + 1).clip(max=G - 1)
        dh, dw = hi - hf, wi - wf
        rows = lambda a, b: table[(a[:, None] * G + b[None, :]).reshape(-1).long()]  # noqa: E731
        emb = (rows(hf, wf) * ((1 - dh)[:, None] * (1 - dw)[None, :]).reshape(-1, 1)
               + rows(hf, wc) * ((1 - dh)[:, None] * dw[None, :]).reshape(-1, 1)
               + rows(hc, wf) * (dh[:, None] * (1 - dw)[None, :]).reshape(-1, 1)
               + rows(hc, wc) * (dh[:, None] * dw[None, :]).reshape(-1, 1))
        emb = emb.repeat(t, 1).view(t, h // merge, merge, w // merge, merge, -1).permute(0, 1, 3, 2, 4, 5)
        out.append(emb.reshape(t * h * w, -1))
    return torch.cat(out)


def vision_tower(patches, p, grid_thw, *, num_heads: int, merge: int, in_channels: int, temporal: int, patch: int,
                 theta: float = 10000.0, eps: float = 1e-6, deepstack_layers=(), per_frame: bool = True, rd=_ident):
    """CudaVisionTower.forward, models/common.py:176-212: patch embed + interpolated position
    embedding, 2D rotary tables, the blocks, deepstack mergers after the listed blocks, the merger.

    per_frame=True: every frame of every image attends only within itself (HF's
    cu_seqlens attention); per_frame=False: one sequence over all images, as the
    reference's forward runs it (models/common.py:198). Returns (pooler_output,
    last_hidden_state, [deepstack features]).
    """
    grids = [tuple(int(v) for v in g) for g in grid_thw]
    x = rd(patch_embed(patches, p["patch_embed.weight"], p["patch_embed.bias"], in_channels, temporal, patch))
    x = rd(x + pos_embed_interpolate(p["pos_embed.emb.weight"], grids, merge))
    hd = x.shape[-1] // num_heads
    cos, sin = vision_rope_tables(grids, hd, theta, merge)
    lens = [h * w for t, h, w in grids for _ in range(t)] if per_frame else [x.shape[0]]
    bounds = [0]
    for n in lens:
        bounds.append(bounds[-1] + n)
    deep = []
    for i in range(len({k.split(".")[1] for k in p if k.startswith("blocks.")})):
        bp = {k[len(f"blocks.{i}."):]: v for k, v in p.items() if k.startswith(f"blocks.{i}.")}
        x = torch.cat([vision_block(x[None, a:b], bp, num_heads=num_heads, cos=cos[a:b], sin=sin[a:b], eps=eps,
                                    rd=rd)[0] for a, b in zip(bounds[:-1], bounds[1:])])
        if i in deepstack_layers:
            j = list(deepstack_layers).index(i)
            deep.append(patch_merger(x, p, merge=merge, postshuffle=True, prefix=f"deepstack_mergers.{j}.", rd=rd))
    return patch_merger(x, p, merge=merge, postshuffle=False, prefix="merger.", rd=rd), x, deep


def text_model(x_embeds, p, *, num_heads, num_kv_heads, head_dim, eps, theta, mrope_section, positions,
               past_kvs=None, visual_pos_masks=None, deepstack_embeds=None, use_moe=None, top_k=0, rd=_ident):
    """CudaQwen3VLDenseModel._text_forward + lm_head, models/dense.py:57-75, 115-118: the layers
    (past_kv each), deepstack adds after the first layers, the final RMSNorm, lm_head.
    p holds the model's text parameters ("layers.N.*", "norm.weight", "lm_head.weight").
    Returns (logits, [(k, v)] per layer)."""
    n_layers = len({k.split(".")[1] for k in p if k.startswith("layers.")})
    cos3, sin3 = ops.mrope_cos_sin(positions, head_dim, theta)
    x, kvs = x_embeds, []
    n_ds = len(deepstack_embeds) if deepstack_embeds is not None else 0
    for i in range(n_layers):
        lp = {k[len(f"layers.{i}."):]: v for k, v in p.items() if k.startswith(f"layers.{i}.")}
        moe = use_moe(i) if use_moe is not None else False
        x, _, kv = text_decoder_layer(x, lp, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                                      eps=eps, cos_3d=cos3, sin_3d=sin3, mrope_section=mrope_section, use_moe=moe,
                                      top_k=top_k, past_kv=past_kvs[i] if past_kvs is not None else None, rd=rd)
        kvs.append(kv)
        if visual_pos_masks is not None and i < n_ds:
            x = x.clone()
            x[visual_pos_masks] = rd(x[visual_pos_masks] + deepstack_embeds[i])
    h = rd(ops.rmsnorm(x, p["norm.weight"], eps))
    return rd(ops.linear(h, p["lm_head.weight"])), kvs


def greedy_generate(input_ids, p, *, max_new_tokens, num_heads, num_kv_heads, head_dim, eps, theta, mrope_section,
                    rd=_ident):
    """CudaQwen3VLDenseModel.generate, models/dense.py:123-162: prefill, then one token at a time
    with the grown (k, v) caches at position past_len, argmax of the last logits.
    Returns (B, S + max_new_tokens) token ids."""
    B, S = input_ids.shape
    kw = dict(num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim, eps=eps, theta=theta,
              mrope_section=mrope_section, rd=rd)
    pos = torch.arange(S).view(1, 1, S).expand(3, B, S)
    logits, kvs = text_model(p["embed_tokens.weight"][input_ids], p, positions=pos, **kw)
    tok = logits[:, -1].argmax(-1, keepdim=True)
    out = torch.cat([input_ids, tok], dim=1)
    for _ in range(max_new_tokens - 1):
        past = kvs[0][0].shape[2]
        pos = torch.full((3, B, 1), past)
        logits, kvs = text_model(p["embed_tokens.weight"][tok], p, positions=pos, past_kvs=kvs, **kw)
        tok = logits[:, -1].argmax(-1, keepdim=True)
        out = torch.cat([out, tok], dim=1)
    return out
