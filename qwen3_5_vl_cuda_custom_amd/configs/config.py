"""Qwen3-VL configuration: the field names and defaults of the reference's configs/config.py:8-55,
and the normalisation of a HuggingFace Qwen3VLConfig / Qwen3VLMoeConfig (config.py:57-120)."""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any


@dataclass
class VisionConfig:
    hidden_size: int = 1152
    num_layers: int = 27
    num_heads: int = 16
    intermediate_size: int = 4304
    patch_size: int = 16
    temporal_patch_size: int = 2
    spatial_merge_size: int = 2
    in_channels: int = 3
    num_position_embeddings: int = 2304
    out_hidden_size: int = 3584
    rope_theta: float = 10000.0
    rms_norm_eps: float = 1e-6
    deepstack_layers: tuple[int, ...] = (8, 16, 24)


@dataclass
class TextConfig:
    hidden_size: int = 4096
    intermediate_size: int = 22016
    num_layers: int = 32
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    vocab_size: int = 151936
    max_position_embeddings: int = 128000
    rope_theta: float = 500000.0
    rms_norm_eps: float = 1e-6
    mrope_section: list[int] = field(default_factory=lambda: [24, 20, 20])
    attention_bias: bool = False
    tie_word_embeddings: bool = False


@dataclass
class MoETextConfig(TextConfig):
    num_experts: int = 60
    num_experts_per_tok: int = 4
    moe_intermediate_size: int = 1408
    norm_topk_prob: bool = True
    decoder_sparse_step: int = 1
    mlp_only_layers: list[int] = field(default_factory=list)


def _get(d: dict, *names, default=None):
    for n in names:
        v = d.get(n)
        if v is not None:
            return v
    return default


@dataclass
class Qwen3VLConfig:
    family: str  # "dense" or "moe"
    vision: VisionConfig
    text: TextConfig | MoETextConfig

    @classmethod
    def from_hf_config(cls, hf_config: Any) -> "Qwen3VLConfig":
        """Our layout from a HuggingFace config object or its dict."""
        raw = hf_config.to_dict() if hasattr(hf_config, "to_dict") else dict(hf_config)
        vr = raw.get("vision_config", {}) or {}
        tr = raw.get("text_config", raw) or {}
        n_exp = int(_get(tr, "num_local_experts", "num_experts", default=0) or 0)
        moe = raw.get("model_type") == "qwen3_vl_moe" or n_exp > 0
        vision = VisionConfig(
            hidden_size=int(_get(vr, "hidden_size", default=1152)),
            num_layers=int(_get(vr, "num_hidden_layers", "depth", default=27)),
            num_heads=int(_get(vr, "num_heads", default=16)),
            intermediate_size=int(_get(vr, "intermediate_size", default=4304)),
            patch_size=int(_get(vr, "patch_size", default=16)),
            temporal_patch_size=int(_get(vr, "temporal_patch_size", default=2)),
            spatial_merge_size=int(_get(vr, "spatial_merge_size", default=2)),
            in_channels=int(_get(vr, "in_channels", default=3)),
            num_position_embeddings=int(_get(vr, "num_position_embeddings", default=2304)),
            out_hidden_size=int(_get(vr, "out_hidden_size", default=None) or _get(tr, "hidden_size", default=3584)),
            rope_theta=float(_get(vr, "rope_theta", default=10000.0)),
            rms_norm_eps=float(_get(vr, "rms_norm_eps", default=1e-6)),
            deepstack_layers=tuple(_get(vr, "deepstack_visual_indexes", default=(8, 16, 24))),
        )
        hidden = int(_get(tr, "hidden_size", default=4096))
        heads = int(_get(tr, "num_attention_heads", default=32))
        rope_scaling = _get(tr, "rope_scaling", "rope_parameters", default={}) or {}
        text_kw = dict(
            hidden_size=hidden,
            intermediate_size=int(_get(tr, "intermediate_size", default=22016)),
            num_layers=int(_get(tr, "num_hidden_layers", default=32)),
            num_heads=heads,
            num_kv_heads=int(_get(tr, "num_key_value_heads", default=8)),
            head_dim=int(_get(tr, "head_dim", default=hidden // heads)),
            vocab_size=int(_get(tr, "vocab_size", default=151936)),
            max_position_embeddings=int(_get(tr, "max_position_embeddings", default=128000)),
            rope_theta=float(_get(tr, "rope_theta", default=None) or rope_scaling.get("rope_theta", 500000.0)),
            rms_norm_eps=float(_get(tr, "rms_norm_eps", default=1e-6)),
            mrope_section=list(rope_scaling.get("mrope_section", [24, 20, 20])),
            attention_bias=bool(_get(tr, "attention_bias", default=False)),
            tie_word_embeddings=bool(_get(raw, "tie_word_embeddings", default=False)),
        )
        if moe:
            text = MoETextConfig(**text_kw, num_experts=n_exp or 60,
                                 num_experts_per_tok=int(_get(tr, "num_experts_per_tok", default=4)),
                                 moe_intermediate_size=int(_get(tr, "moe_intermediate_size", default=1408)),
                                 norm_topk_prob=bool(_get(tr, "norm_topk_prob", default=True)),
                                 decoder_sparse_step=int(_get(tr, "decoder_sparse_step", default=1)),
                                 mlp_only_layers=list(_get(tr, "mlp_only_layers", default=[]) or []))
        else:
            text = TextConfig(**text_kw)
        return cls(family="moe" if moe else "dense", vision=vision, text=text)
