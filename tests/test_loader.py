"""The HF checkpoint loader and config normalisation on the CPU (reference loaders/hf.py:21-109,
configs/config.py:57-120): HF's own tiny models define the checkpoint names; every one of them
must land on a parameter of the model classes, with the MoE expert matrices transposed from
their on-disk layout."""
import pytest
import torch

from qwen3_5_vl_cuda_custom_amd.configs import MoETextConfig, Qwen3VLConfig
from qwen3_5_vl_cuda_custom_amd.loaders import load_hf_weights, map_hf_name
from qwen3_5_vl_cuda_custom_amd.models import CudaQwen3VLDenseModel, CudaQwen3VLMoeModel

TEXT = dict(hidden_size=32, intermediate_size=48, num_attention_heads=2, num_key_value_heads=1, head_dim=16,
            num_hidden_layers=2, vocab_size=40,
            rope_parameters={"rope_type": "default", "rope_theta": 1e4, "mrope_section": [4, 2, 2]})
VISION = dict(depth=2, hidden_size=32, num_heads=2, intermediate_size=48, patch_size=4, out_hidden_size=32,
              num_position_embeddings=16, deepstack_visual_indexes=[0])


def _save(state: dict, path, transpose_experts=False):
    from safetensors.torch import save_file
    out = {}
    for k, t in state.items():
        t = t.detach().clone()
        if transpose_experts and ("mlp.experts.gate_up_proj" in k or "mlp.experts.down_proj" in k):
            t = t.transpose(1, 2).contiguous()  # the checkpoint's (E, H, 2I) / (E, I, H) layout
        out[k] = t.contiguous()
    half = len(out) // 2
    keys = sorted(out)
    save_file({k: out[k] for k in keys[:half]}, str(path / "model-00001-of-00002.safetensors"))
    save_file({k: out[k] for k in keys[half:]}, str(path / "model-00002-of-00002.safetensors"))


def _randomise(model, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for prm in model.parameters():
            prm.copy_(torch.randn(prm.shape, generator=g))


def test_dense_checkpoint_names_all_land(tmp_path):
    from transformers.models.qwen3_vl import modeling_qwen3_vl as M
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLConfig as HFConfig
    hcfg = HFConfig(text_config=TEXT, vision_config=VISION)
    hf = M.Qwen3VLForConditionalGeneration(hcfg)
    _randomise(hf, 1)
    _save(hf.state_dict(), tmp_path)
    cfg = Qwen3VLConfig.from_hf_config(hcfg)
    assert cfg.family == "dense" and cfg.text.num_layers == 2 and cfg.vision.num_layers == 2
    assert cfg.text.mrope_section == [4, 2, 2] and cfg.vision.deepstack_layers == (0,)
    model = CudaQwen3VLDenseModel(cfg)
    rep = load_hf_weights(model, tmp_path)
    assert rep["missing"] == [] and rep["unexpected"] == [] and rep["mismatched"] == [], rep
    hs = hf.state_dict()
    ours = model.state_dict()
    for k, t in hs.items():
        assert torch.equal(ours[map_hf_name(k)], t), k


def test_moe_checkpoint_experts_transposed(tmp_path):
    from transformers.models.qwen3_vl_moe import modeling_qwen3_vl_moe as MM
    from transformers.models.qwen3_vl_moe.configuration_qwen3_vl_moe import Qwen3VLMoeConfig
    hcfg = Qwen3VLMoeConfig(text_config=dict(TEXT, moe_intermediate_size=24, num_experts=4, num_experts_per_tok=2),
                            vision_config=VISION)
    hf = MM.Qwen3VLMoeForConditionalGeneration(hcfg)
    _randomise(hf, 2)
    _save(hf.state_dict(), tmp_path, transpose_experts=True)
    cfg = Qwen3VLConfig.from_hf_config(hcfg)
    assert cfg.family == "moe" and isinstance(cfg.text, MoETextConfig) and cfg.text.num_experts == 4
    model = CudaQwen3VLMoeModel(cfg)
    rep = load_hf_weights(model, tmp_path)
    assert rep["missing"] == [] and rep["unexpected"] == [] and rep["mismatched"] == [], rep
    ours = model.state_dict()
    for k, t in hf.state_dict().items():  # HF's in-memory layout is the model's: (E, 2I, H), (E, H, I)
        assert torch.equal(ours[map_hf_name(k)], t), k
    assert ours["layers.0.mlp.gate_up_proj"].shape == (4, 48, 32)


def test_name_map_and_missing_snapshot(tmp_path):
    assert map_hf_name("model.visual.patch_embed.proj.weight") == "visual.patch_embed.weight"
    assert map_hf_name("model.visual.pos_embed.weight") == "visual.pos_embed.emb.weight"
    assert map_hf_name("model.visual.deepstack_merger_list.1.norm.bias") == "visual.deepstack_mergers.1.norm.bias"
    assert map_hf_name("model.language_model.layers.3.mlp.gate.weight") == "layers.3.mlp.gate_weight"
    assert map_hf_name("lm_head.weight") == "lm_head.weight"
    assert map_hf_name("something.else") is None
    with pytest.raises(FileNotFoundError):
        load_hf_weights(torch.nn.Linear(2, 2), tmp_path)
