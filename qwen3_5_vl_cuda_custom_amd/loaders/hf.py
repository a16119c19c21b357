"""Load a HuggingFace Qwen3-VL safetensors snapshot into the model classes
(reference loaders/hf.py:21-109: the same key mapping and MoE expert transpose).

HF keys and the module names they land on:
  lm_head.weight                                 lm_head.weight
  model.language_model.<rest>                    <rest>, with (MoE) mlp.experts.gate_up_proj ->
                                                 mlp.gate_up_proj, mlp.experts.down_proj -> mlp.down_proj,
                                                 mlp.gate.weight -> mlp.gate_weight
  model.visual.patch_embed.proj.{weight,bias}    visual.patch_embed.{weight,bias}
  model.visual.pos_embed.weight                  visual.pos_embed.emb.weight
  model.visual.deepstack_merger_list.N.<rest>    visual.deepstack_mergers.N.<rest>
  model.visual.<rest>                            visual.<rest>
HF stores the MoE expert matrices transposed on their last two dims
(gate_up (E, H, 2I), down (E, I, H)); they are transposed on load to
(E, 2I, H) and (E, H, I). Safetensors only: nothing is unpickled.
"""
from __future__ import annotations

from pathlib import Path

import torch

_VISUAL_RENAMES = (("patch_embed.proj.", "patch_embed."), ("deepstack_merger_list.", "deepstack_mergers."))
_TEXT_RENAMES = (("mlp.experts.gate_up_proj", "mlp.gate_up_proj"), ("mlp.experts.down_proj", "mlp.down_proj"),
                 ("mlp.gate.weight", "mlp.gate_weight"))
_TRANSPOSED = ("mlp.experts.gate_up_proj", "mlp.experts.down_proj")


def map_hf_name(name: str) -> str | None:
    """The module name an HF key loads into, or None for keys this model does not hold."""
    if name == "lm_head.weight":
        return name
    if name.startswith("model.visual."):
        rest = name[len("model.visual."):]
        if rest == "pos_embed.weight":
            return "visual.pos_embed.emb.weight"
        for a, b in _VISUAL_RENAMES:
            rest = rest.replace(a, b)
        return "visual." + rest
    if name.startswith("model.language_model."):
        rest = name[len("model.language_model."):]
        for a, b in _TEXT_RENAMES:
            rest = rest.replace(a, b)
        return rest
    return None


def _needs_transpose(name: str) -> bool:
    return any(k in name for k in _TRANSPOSED)


def load_hf_weights(model: torch.nn.Module, snapshot_path: str | Path) -> dict:
    """Copy every mapped tensor of the snapshot's *.safetensors into the model's parameters and
    buffers (cast to their dtype and device). Returns {'loaded', 'missing', 'unexpected', 'mismatched'}."""
    from safetensors import safe_open

    files = sorted(Path(snapshot_path).glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no .safetensors files in {snapshot_path}")
    state = dict(model.state_dict())
    remaining = set(state)
    loaded, unexpected, mismatched = [], [], []
    for f in files:
        with safe_open(str(f), framework="pt", device="cpu") as sf:
            for key in sf.keys():
                target_name = map_hf_name(key)
                if target_name is None or target_name not in state:
                    unexpected.append(key)
                    continue
                t = sf.get_tensor(key)
                if _needs_transpose(key):
                    t = t.transpose(1, 2).contiguous()
                target = state[target_name]
                if tuple(t.shape) != tuple(target.shape):
                    mismatched.append((key, tuple(t.shape), tuple(target.shape)))
                    continue
                with torch.no_grad():
                    target.copy_(t.to(dtype=target.dtype, device=target.device))
                loaded.append(target_name)
                remaining.discard(target_name)
    return {"loaded": loaded, "missing": sorted(remaining), "unexpected": unexpected, "mismatched": mismatched}
