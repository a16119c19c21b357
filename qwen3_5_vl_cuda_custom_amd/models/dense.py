"""CudaQwen3VLDenseModel (reference models/dense.py:18-162): vision tower + text decoder stack
+ lm_head, with the reference's `past_key_values` forward and a batched greedy `generate`.

`generate` keeps the reference's call form and results for equal-length
prompts and adds what a serving loop needs: ragged prompts (`prompt_lens`,
right-padded `input_ids`), per-sequence positions (each sequence decodes at
its own length, plus an optional mRoPE delta), a preallocated KV cache per
layer (StaticKVCache, appended in place) and the per-token step captured once
as a HIP graph and replayed (the reference grows every layer's cache with
torch.cat and launches every op from Python, models/dense.py:148-152).
"""
from __future__ import annotations

import torch
from torch import nn

from ..configs import Qwen3VLConfig
from ..kernels import cuda_index_add
from ..modules import (CudaEmbedding, CudaLinear, CudaRMSNorm, CudaTextDecoderLayer, PagedKVCache, StaticKVCache,
                       StepGraph,
                       TextMRoPE)
from .common import CudaVisionTower


def text_positions(position_ids, batch: int, seq: int, past_len: int, device) -> torch.Tensor:
    """(3, B, S) positions from the reference's accepted forms (models/dense.py:97-108):
    None -> past_len + arange(S) on every axis; (3, B, S); (4, B, S) -> its last three."""
    if position_ids is None:
        pos = torch.arange(past_len, past_len + seq, device=device).unsqueeze(0).expand(batch, seq)
        return torch.stack([pos, pos, pos], dim=0)
    if position_ids.dim() == 3 and position_ids.shape[0] == 4:
        return position_ids[1:]
    if position_ids.dim() == 3 and position_ids.shape[0] == 3:
        return position_ids
    raise ValueError(f"Unsupported position_ids shape {tuple(position_ids.shape)}")


class _TextLM(nn.Module):
    """The text side shared by the dense and MoE models: embeddings, layers, norm, lm_head."""

    cfg: Qwen3VLConfig
    embed_tokens: CudaEmbedding
    rotary: TextMRoPE
    layers: nn.ModuleList
    norm: CudaRMSNorm
    lm_head: CudaLinear

    def _init_text(self, t, layer_uses_moe) -> None:
        self.embed_tokens = CudaEmbedding(t.vocab_size, t.hidden_size)
        self.rotary = TextMRoPE(t.head_dim, theta=t.rope_theta, mrope_section=t.mrope_section)
        self.layers = nn.ModuleList([
            CudaTextDecoderLayer(hidden_size=t.hidden_size, num_heads=t.num_heads, num_kv_heads=t.num_kv_heads,
                                 head_dim=t.head_dim, intermediate_size=t.intermediate_size,
                                 rms_norm_eps=t.rms_norm_eps, use_moe=layer_uses_moe(i),
                                 num_experts=getattr(t, "num_experts", 0), top_k=getattr(t, "num_experts_per_tok", 0),
                                 moe_intermediate_size=getattr(t, "moe_intermediate_size", 0),
                                 attention_bias=t.attention_bias)
            for i in range(t.num_layers)])
        self.norm = CudaRMSNorm(t.hidden_size, eps=t.rms_norm_eps)
        self.lm_head = CudaLinear(t.hidden_size, t.vocab_size, bias=False)
        if t.tie_word_embeddings:
            self.lm_head.weight = self.embed_tokens.weight

    def _deepstack_process(self, hidden_states: torch.Tensor, visual_pos_masks: torch.Tensor,
                           visual_embeds: torch.Tensor) -> torch.Tensor:
        """hidden[mask] += visual_embeds (models/dense.py:46-55): an index_add over the visual
        positions (unique, so each is one bf16 add), on a copy as the reference does."""
        H = hidden_states.shape[-1]
        idx = visual_pos_masks.to(hidden_states.device).reshape(-1).nonzero().squeeze(1)
        out = hidden_states.reshape(-1, H).clone()
        cuda_index_add(out, visual_embeds.to(device=out.device, dtype=out.dtype).reshape(-1, H), idx)
        return out.view_as(hidden_states)

    def _run_layers(self, x, binding, visual_pos_masks=None, deepstack_visual_embeds=None, past_key_values=None,
                    caches=None, router_logits=None):
        n_ds = len(deepstack_visual_embeds) if deepstack_visual_embeds is not None else 0
        new_kvs = []
        for i, layer in enumerate(self.layers):
            past = past_key_values[i] if past_key_values is not None else None
            cache = caches[i] if caches is not None else None
            x, rl, kv = layer(x, binding, past_kv=past, kv_cache=cache)
            if router_logits is not None and rl is not None:
                router_logits.append(rl)
            new_kvs.append(kv)
            if visual_pos_masks is not None and i < n_ds:
                x = self._deepstack_process(x, visual_pos_masks, deepstack_visual_embeds[i])
        return self.norm(x), new_kvs

    # ------------------------------------------------------------ KV-cache serving path
    def new_caches(self, batch: int, capacity: int, device=None, dtype=None, *, page_rows: int = 0,
                   num_pages: int | None = None) -> list[StaticKVCache] | list[PagedKVCache]:
        """One cache per layer, empty, for `batch` sequences of up to `capacity` tokens: a StaticKVCache,
        or with page_rows > 0 a PagedKVCache of `num_pages` pages (default: enough for every sequence
        to reach `capacity`)."""
        t = self.cfg.text
        dev = device if device is not None else self.lm_head.weight.device
        dt = dtype if dtype is not None else self.lm_head.weight.dtype
        if page_rows > 0:
            per_seq = -(-capacity // page_rows)
            n = num_pages if num_pages is not None else batch * per_seq
            return [PagedKVCache(batch, t.num_kv_heads, t.head_dim, num_pages=n, max_pages=per_seq,
                                 page_rows=page_rows, dtype=dt, device=dev) for _ in range(t.num_layers)]
        return [StaticKVCache(batch, t.num_kv_heads, capacity, t.head_dim, dtype=dt, device=dev)
                for _ in range(t.num_layers)]

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int = 32, eos_token_id: int | None = None,
                 position_ids: torch.Tensor | None = None, visual_pos_masks: torch.Tensor | None = None,
                 deepstack_visual_embeds: list[torch.Tensor] | None = None,
                 inputs_embeds: torch.Tensor | None = None, *, prompt_lens=None,
                 rope_deltas: torch.Tensor | None = None, use_graph: bool = True,
                 page_rows: int = 0) -> torch.Tensor:
        """Greedy decoding (reference models/dense.py:123-162). Returns (B, S + new tokens):
        each row's prompt (as given, padding included) followed by its generated tokens.

        prompt_lens: per-sequence prompt lengths for right-padded `input_ids`
        (default: all S). rope_deltas (B,): added to a sequence's cache length
        to give its decode position (the mRoPE offset after images; default 0).
        Generation stops early only when every sequence has just produced
        `eos_token_id`, as in the reference. page_rows > 0 keeps the KV cache
        in pages of that many rows (a multiple of 32) instead of one
        preallocated block per sequence.
        """
        B, S = input_ids.shape
        dev = self.lm_head.weight.device
        lens = [int(v) for v in prompt_lens] if prompt_lens is not None else [S] * B
        if len(lens) != B or min(lens) < 1 or max(lens) > S:
            raise ValueError("generate: prompt_lens must give 1..S tokens for every sequence")
        caches = self.new_caches(B, S + max_new_tokens, dev, page_rows=page_rows)
        emb = inputs_embeds if inputs_embeds is not None else self.embed_tokens(input_ids.to(dev))
        pos3 = text_positions(position_ids, B, S, 0, dev)
        h, _ = self._run_layers(emb, self.rotary.bind(pos3), visual_pos_masks, deepstack_visual_embeds,
                                caches=caches)
        last = h[torch.arange(B, device=dev), torch.tensor(lens, device=dev) - 1]  # each prompt's last token
        tok = self.lm_head(last).argmax(-1).view(B, 1)
        for c in caches:  # padded rows past a prompt are dropped (overwritten by the decode tokens)
            c.set_lens(lens)
        out = [tok.clone()]
        if max_new_tokens <= 1:
            return torch.cat([input_ids.to(dev), tok], dim=1)

        delta = (rope_deltas.to(device=dev, dtype=torch.int32) if rope_deltas is not None
                 else torch.zeros(B, dtype=torch.int32, device=dev))
        pos32 = torch.empty(3, B, 1, dtype=torch.int32, device=dev)
        binding = self.rotary.bind(pos32)

        def step():
            pos32.copy_((caches[0].lens + delta).view(1, B, 1).expand(3, B, 1))
            hs, _ = self._run_layers(self.embed_tokens(tok), binding, caches=caches)
            tok.copy_(self.lm_head(hs[:, -1]).argmax(-1).view(B, 1))
            return tok

        graph = None
        for n in range(1, max_new_tokens):
            if eos_token_id is not None and bool((tok == eos_token_id).all()):
                break
            if graph is not None:
                graph.replay()
            else:
                step()
                if use_graph and n + 1 < max_new_tokens:
                    graph = StepGraph(step, warmup=0, caches=caches)  # capture only: nothing runs
            out.append(tok.clone())
        return torch.cat([input_ids.to(dev), *out], dim=1)


class CudaQwen3VLDenseModel(_TextLM):
    """Dense Qwen3-VL: `visual`, `embed_tokens`, `rotary`, `layers`, `norm`, `lm_head` (the reference's names)."""

    def __init__(self, cfg: Qwen3VLConfig) -> None:
        super().__init__()
        if cfg.family != "dense":
            raise ValueError(f"expected a dense config, got {cfg.family}")
        self.cfg = cfg
        self.visual = CudaVisionTower(cfg.vision)
        self._init_text(cfg.text, lambda i: False)

    def forward(self, input_ids: torch.Tensor | None = None, inputs_embeds: torch.Tensor | None = None,
                position_ids: torch.Tensor | None = None, visual_pos_masks: torch.Tensor | None = None,
                deepstack_visual_embeds: list[torch.Tensor] | None = None,
                past_key_values: list[tuple[torch.Tensor, torch.Tensor]] | None = None, return_kv: bool = False):
        """Logits (B, S, vocab) (and the grown per-layer (k, v) with return_kv), models/dense.py:77-120."""
        if (input_ids is None) == (inputs_embeds is None):
            raise ValueError("Specify exactly one of input_ids / inputs_embeds")
        if inputs_embeds is None:
            inputs_embeds = self.embed_tokens(input_ids)
        B, S = inputs_embeds.shape[:2]
        past_len = past_key_values[0][0].shape[2] if past_key_values else 0
        pos3 = text_positions(position_ids, B, S, past_len, inputs_embeds.device)
        hidden, new_kvs = self._run_layers(inputs_embeds, self.rotary.bind(pos3), visual_pos_masks,
                                           deepstack_visual_embeds, past_key_values=past_key_values)
        logits = self.lm_head(hidden)
        return (logits, new_kvs) if return_kv else logits
