"""CudaQwen3VLMoeModel (reference models/moe.py:26-105): the text stack with sparse-MoE MLPs
(on the layers `decoder_sparse_step` selects, except `mlp_only_layers`)."""
from __future__ import annotations

import torch

from ..configs import MoETextConfig, Qwen3VLConfig
from .common import CudaVisionTower
from .dense import _TextLM, text_positions


def layer_uses_moe(cfg: MoETextConfig, layer_idx: int) -> bool:
    """models/moe.py:18-23."""
    if cfg.num_experts <= 0 or layer_idx in cfg.mlp_only_layers:
        return False
    return (layer_idx + 1) % cfg.decoder_sparse_step == 0


class CudaQwen3VLMoeModel(_TextLM):
    """MoE Qwen3-VL: `visual`, `embed_tokens`, `rotary`, `layers`, `norm`, `lm_head`."""

    def __init__(self, cfg: Qwen3VLConfig) -> None:
        super().__init__()
        if cfg.family != "moe" or not isinstance(cfg.text, MoETextConfig):
            raise ValueError(f"expected an MoE config, got {cfg.family}")
        self.cfg = cfg
        self.visual = CudaVisionTower(cfg.vision)
        self._init_text(cfg.text, lambda i: layer_uses_moe(cfg.text, i))

    def forward(self, input_ids: torch.Tensor, pixel_values: torch.Tensor | None = None,
                vision_position_ids: torch.Tensor | None = None, image_token_mask: torch.Tensor | None = None,
                position_ids: torch.Tensor | None = None,
                past_key_values: list[tuple[torch.Tensor, torch.Tensor]] | None = None, return_kv: bool = False):
        """(logits, router_logits per MoE layer) (+ new (k, v) per layer with return_kv), models/moe.py:72-105.

        Image features replace the embeddings at `image_token_mask`
        (vision_position_ids: the images' (t, h, w) grid). The tower's pooled
        output is used; the reference unpacks the tower's three outputs into
        two there, which raises.
        """
        inputs_embeds = self.embed_tokens(input_ids)
        if pixel_values is not None and image_token_mask is not None:
            feats = self.visual(pixel_values, vision_position_ids)[0]
            inputs_embeds = inputs_embeds.clone()
            inputs_embeds[image_token_mask] = feats.to(inputs_embeds.dtype)
        B, S = input_ids.shape
        past_len = past_key_values[0][0].shape[2] if past_key_values else 0
        pos3 = text_positions(position_ids, B, S, past_len, inputs_embeds.device)
        router_logits: list[torch.Tensor] = []
        hidden, new_kvs = self._run_layers(inputs_embeds, self.rotary.bind(pos3), past_key_values=past_key_values,
                                           router_logits=router_logits)
        logits = self.lm_head(hidden)
        return (logits, router_logits, new_kvs) if return_kv else (logits, router_logits)
