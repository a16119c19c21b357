"""Writes tests/golden/c1_layer.npz: the C1 tiny decoder layer's output from HF transformers.

The C1 case (hidden 256, 4q/2kv heads x 64, I 688, mrope [12,10,10], theta 5e6,
S 128, fp32) is built from a seeded CPU generator, so only its output and an
input checksum are stored. The expected output comes from transformers'
Qwen3VLTextDecoderLayer (an implementation independent of the reference and of
this repository's oracle), run in fp32 with eager attention and a causal mask.

Run: python -m tests.golden.make_golden
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
NAMES = ["input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_proj.weight",
         "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
         "self_attn.q_norm.weight", "self_attn.k_norm.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
         "mlp.down_proj.weight"]
SHAPES = {"input_layernorm.weight": (256,), "post_attention_layernorm.weight": (256,),
          "self_attn.q_proj.weight": (256, 256), "self_attn.k_proj.weight": (128, 256),
          "self_attn.v_proj.weight": (128, 256), "self_attn.o_proj.weight": (256, 256),
          "self_attn.q_norm.weight": (64,), "self_attn.k_norm.weight": (64,),
          "mlp.gate_proj.weight": (688, 256), "mlp.up_proj.weight": (688, 256), "mlp.down_proj.weight": (256, 688)}


def c1_case(seed: int = 0):
    """x (1, 128, 256) N(0,1), positions (3, 1, 128), params: matrices N(0, 0.02), norm weights 1 + 0.1 N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    p = {}
    for n in NAMES:
        shape = SHAPES[n]
        p[n] = torch.randn(shape, generator=g) * 0.02 if len(shape) == 2 else 1 + 0.1 * torch.randn(shape, generator=g)
    x = torch.randn(1, 128, 256, generator=g)
    pos = torch.arange(128).view(1, 1, 128).expand(3, 1, 128)
    return x, pos, p


def hf_c1_output(x, pos, p):
    from transformers.models.qwen3_vl import modeling_qwen3_vl as M
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    cfg = Qwen3VLTextConfig(hidden_size=256, intermediate_size=688, num_attention_heads=4, num_key_value_heads=2,
                            head_dim=64, rms_norm_eps=1e-6,
                            rope_parameters={"rope_type": "default", "rope_theta": 5e6, "mrope_section": [12, 10, 10]})
    cfg._attn_implementation = "eager"
    layer = M.Qwen3VLTextDecoderLayer(cfg, 0).eval()
    layer.load_state_dict(p)
    cos, sin = M.Qwen3VLTextRotaryEmbedding(cfg)(x, pos)
    mask = torch.full((128, 128), float("-inf")).triu(1)[None, None]
    with torch.no_grad():
        return layer(x, (cos, sin), attention_mask=mask)


def load_fixture(name: str):
    with np.load(HERE / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def main():
    x, pos, p = c1_case()
    y = hf_c1_output(x, pos, p)
    np.savez_compressed(HERE / "c1_layer.npz", y=y.numpy().astype(np.float32), x_sum=np.float64(x.double().sum()))
    print("wrote", HERE / "c1_layer.npz", tuple(y.shape))


if __name__ == "__main__":
    main()
