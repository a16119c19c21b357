"""GPU parity of the model-edge and vision-tower rows: embedding, GELU-fused GEMM, packed
variable-length attention, the vision rotary / position-embedding kernels, the patch merger,
the whole vision tower, the dense / MoE model forwards and the batched greedy decode loop.
Everything is compared with the CPU-restated oracle (fp32) on the same seeded inputs."""
import pytest
import torch

from oracle import layers as L
from oracle import ops as O
from qwen3_5_vl_cuda_custom_amd import kernels as K
from qwen3_5_vl_cuda_custom_amd import workloads as W
from qwen3_5_vl_cuda_custom_amd.configs import MoETextConfig, Qwen3VLConfig, TextConfig, VisionConfig
from qwen3_5_vl_cuda_custom_amd.models import CudaQwen3VLDenseModel, CudaQwen3VLMoeModel, CudaVisionTower
from qwen3_5_vl_cuda_custom_amd.modules import CudaVisionPatchMerger
from tests.parity import assert_bf16_close, assert_close, assert_layer_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rnd(*shape, seed=0, std=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def params(module, device="cpu", prefix=""):
    return {n[len(prefix):]: t.detach().float().to(device) for n, t in module.state_dict().items()
            if n.startswith(prefix)}


# ------------------------------------------------------------------ ops
def test_embedding_gather_and_bad_ids():
    from qwen3_5_vl_cuda_custom_amd import _lib
    _lib.device_status(DEV)
    w = rnd(1000, 256, seed=1)
    ids = torch.randint(0, 1000, (3, 17), generator=torch.Generator().manual_seed(2))
    out = K.embedding(ids.to(DEV), w.to(DEV))
    assert out.shape == (3, 17, 256) and torch.equal(out.cpu(), torch.nn.functional.embedding(ids, w))
    K.raise_device_errors(DEV)
    wf = w.float()
    assert torch.equal(K.embedding(ids.to(DEV), wf.to(DEV)).cpu(), torch.nn.functional.embedding(ids, wf))
    odd = rnd(50, 36, seed=3)  # a row length that is not a multiple of 16 bytes' elements
    bad = torch.tensor([0, 49, 50, -1, 7])
    got = K.embedding(bad.to(DEV), odd.to(DEV)).cpu()
    assert torch.equal(got[[0, 1, 4]], odd[[0, 49, 7]]) and torch.equal(got[2:4], torch.zeros(2, 36).bfloat16())
    with pytest.raises(IndexError):
        K.raise_device_errors(DEV)


@pytest.mark.parametrize("M,N,Kd,dt", [(3136, 4304, 1152, torch.bfloat16), (700, 4608, 4608, torch.bfloat16),
                                        (20, 96, 64, torch.bfloat16), (33, 70, 40, torch.float32)])
def test_matmul_gelu(M, N, Kd, dt):
    x, w, b = rnd(M, Kd, seed=4, dtype=dt), rnd(N, Kd, seed=5, std=Kd ** -0.5, dtype=dt), rnd(N, seed=6, dtype=dt)
    y = K.matmul_gelu(x.to(DEV), w.to(DEV), b.to(DEV))
    ref = O.gelu_tanh(O.linear(x.float(), w.float(), b.float()))
    if dt == torch.float32:
        assert_close(y, ref, atol=2e-5, what="matmul_gelu fp32")
    else:
        assert_bf16_close(y, ref, what=f"matmul_gelu {M}x{N}x{Kd}")


@pytest.mark.parametrize("H,Hkv,D,causal,dt", [(16, 16, 72, False, torch.bfloat16), (8, 2, 128, True, torch.bfloat16),
                                                (4, 4, 64, False, torch.bfloat16), (2, 1, 32, True, torch.float32)])
def test_flash_attention_varlen(H, Hkv, D, causal, dt):
    lens = [784, 1, 130, 64, 720, 257]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    T = int(cu[-1])
    q = rnd(H, T, D, seed=7, dtype=dt)
    kv = rnd(2, Hkv, T, D, seed=8, dtype=dt)
    out = K.flash_attention_varlen(q.to(DEV), kv[0].to(DEV), kv[1].to(DEV), cu.to(DEV), max(lens), D ** -0.5,
                                   causal, H // Hkv)
    ref = torch.cat([O.flash_attention(q[None, :, a:b].float(), kv[0][None, :, a:b].float(),
                                       kv[1][None, :, a:b].float(), D ** -0.5, causal, H // Hkv)[0]
                     for a, b in zip(cu[:-1].tolist(), cu[1:].tolist())], dim=1)
    if dt == torch.float32:
        assert_close(out, ref, atol=2e-5, what="varlen fp32")
    else:
        assert_bf16_close(out, ref, what=f"varlen H={H} D={D} causal={causal}")


GRIDS = [(1, 28, 28), (1, 20, 36), (2, 16, 16), (1, 4, 8)]


def test_vision_rope_tables_and_pos_embed():
    hd, merge = 72, 2
    inv = (1.0 / (1e4 ** (torch.arange(0, hd // 2, 2, dtype=torch.float32) / (hd // 2))))
    cos, sin = K.vision_rope_tables(GRIDS, merge, inv.to(DEV), hd)
    rc, rs = L.vision_rope_tables(GRIDS, hd, 1e4, merge)
    assert_close(cos, rc, atol=2e-6, what="vision cos")
    assert_close(sin, rs, atol=2e-6, what="vision sin")
    total = rc.shape[0]
    table = rnd(48 * 48, 1152, seed=9)
    x = rnd(total, 1152, seed=10)
    y = K.vision_pos_embed(x.to(DEV), table.to(DEV), GRIDS, merge)
    ref = x.float() + L.pos_embed_interpolate(table.float(), GRIDS, merge)
    assert_bf16_close(y, ref, what="pos embed + x")
    xd = x.to(DEV)
    K.vision_pos_embed(xd, table.to(DEV), GRIDS, merge, out=xd)  # in place
    assert torch.equal(xd, y)
    with pytest.raises(ValueError):
        K.vision_pos_embed(x.to(DEV), table.to(DEV), [(1, 5, 8)], merge)  # h not a multiple of merge


@pytest.mark.parametrize("post", [False, True])
def test_patch_merger(post):
    m = CudaVisionPatchMerger(1152, 4096, 2, use_postshuffle_norm=post).to(DEV, torch.bfloat16)
    W.init_normal_(m, seed=11, include_bias=True)
    x = rnd(3136, 1152, seed=12).to(DEV)
    y = m(x)
    p = params(m)
    ref = L.patch_merger(x.float().cpu(), p, merge=2, postshuffle=post)
    emu = L.patch_merger(x.float().cpu(), p, merge=2, postshuffle=post, rd=O.round_bf16)
    assert y.shape == (784, 4096)
    assert_layer_parity(y, ref, emu, what=f"patch merger postshuffle={post}")


# ------------------------------------------------------------------ vision tower
def _tower(depth=2, deepstack=(0,), seed=13):
    vc = VisionConfig(num_layers=depth, deepstack_layers=deepstack, out_hidden_size=4096)
    tower = CudaVisionTower(vc).to(DEV, torch.bfloat16)
    W.init_normal_(tower, seed=seed, include_bias=True)
    return vc, tower


def test_vision_tower_ragged_images():
    """Four images of different grids (one of two frames) through patch embed, position
    embedding, two blocks (each frame attending within itself), a deepstack merger and the
    merger, against the oracle tower (per-frame attention; pinned against HF)."""
    vc, tower = _tower()
    n = sum(t * h * w for t, h, w in GRIDS)
    px = (torch.rand(n, 1536, generator=torch.Generator().manual_seed(14)) * 2 - 1).to(torch.bfloat16)
    pool, last, deep = tower(px.to(DEV), torch.tensor(GRIDS))
    p = params(tower)
    kw = dict(num_heads=vc.num_heads, merge=2, in_channels=3, temporal=2, patch=16, deepstack_layers=(0,))
    rp, rl, rd = L.vision_tower(px.float(), p, GRIDS, **kw)
    ep, el, ed = L.vision_tower(px.float(), p, GRIDS, rd=O.round_bf16, **kw)
    assert pool.shape == (n // 4, 4096) and len(deep) == 1
    assert_layer_parity(last, rl, el, what="tower last hidden")
    assert_layer_parity(pool, rp, ep, what="tower pooler")
    assert_layer_parity(deep[0], rd[0], ed[0], what="tower deepstack 0")


# ------------------------------------------------------------------ dense / MoE models
def _text_cfg(**kw):
    base = dict(hidden_size=256, intermediate_size=512, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64,
                vocab_size=1000, rope_theta=1e4, mrope_section=[12, 10, 10])
    base.update(kw)
    return base


def _dense(dtype, seed=15):
    vc = VisionConfig(hidden_size=128, num_layers=1, num_heads=2, intermediate_size=256, patch_size=8,
                      num_position_embeddings=64, out_hidden_size=256, deepstack_layers=(0,))
    cfg = Qwen3VLConfig(family="dense", vision=vc, text=TextConfig(**_text_cfg()))
    m = CudaQwen3VLDenseModel(cfg).to(DEV, dtype)
    W.init_normal_(m, seed=seed, include_bias=True)
    with torch.no_grad():
        m.embed_tokens.weight.normal_(0, 1.0, generator=torch.Generator(device=DEV).manual_seed(seed + 1))
    return m.eval().requires_grad_(False)


def _oracle_kw(m):
    t = m.cfg.text
    return dict(num_heads=t.num_heads, num_kv_heads=t.num_kv_heads, head_dim=t.head_dim, eps=t.rms_norm_eps,
                theta=t.rope_theta, mrope_section=list(t.mrope_section))


def test_dense_forward_with_deepstack_and_past_kv():
    m = _dense(torch.bfloat16)
    B, S = 2, 40
    ids = torch.randint(0, 1000, (B, S), generator=torch.Generator().manual_seed(16))
    mask = torch.zeros(B, S, dtype=torch.bool)
    mask[0, 5:13] = True
    mask[1, 20:24] = True
    ds = [rnd(12, 256, seed=17)]
    logits, kvs = m(input_ids=ids.to(DEV), visual_pos_masks=mask.to(DEV), deepstack_visual_embeds=[ds[0].to(DEV)],
                    return_kv=True)
    p = params(m)
    emb = p["embed_tokens.weight"][ids]
    pos = torch.arange(S).view(1, 1, S).expand(3, B, S)
    kw = dict(positions=pos, visual_pos_masks=mask, deepstack_embeds=[ds[0].float()], **_oracle_kw(m))
    ref, _ = L.text_model(emb, p, **kw)
    emu, _ = L.text_model(emb, p, rd=O.round_bf16, **kw)
    assert_layer_parity(logits, ref, emu, what="dense logits (deepstack)")
    # one more token through the reference's past_kv form
    nxt = torch.randint(0, 1000, (B, 1), generator=torch.Generator().manual_seed(18))
    l2 = m(input_ids=nxt.to(DEV), past_key_values=kvs)
    past = [(k.float().cpu(), v.float().cpu()) for k, v in kvs]
    kw2 = dict(positions=torch.full((3, B, 1), S), past_kvs=past, **_oracle_kw(m))
    r2, _ = L.text_model(p["embed_tokens.weight"][nxt], p, **kw2)
    e2, _ = L.text_model(p["embed_tokens.weight"][nxt], p, rd=O.round_bf16, **kw2)
    assert_layer_parity(l2, r2, e2, what="dense logits (past_kv step)")


def test_generate_fp32_matches_oracle_greedy_and_ragged_prompts():
    """fp32: the batched KV-cache + HIP-graph loop gives the oracle's greedy tokens (the
    reference's past_kv loop); ragged right-padded prompts give each sequence the tokens it
    gets alone."""
    m = _dense(torch.float32)
    ids = torch.randint(0, 1000, (3, 9), generator=torch.Generator().manual_seed(19))
    out = m.generate(ids.to(DEV), max_new_tokens=6)
    ref = L.greedy_generate(ids, params(m), max_new_tokens=6, **_oracle_kw(m))
    assert torch.equal(out.cpu(), ref)
    eager = m.generate(ids.to(DEV), max_new_tokens=6, use_graph=False)
    assert torch.equal(out, eager)
    lens = [9, 4, 7]
    rag = m.generate(ids.to(DEV), max_new_tokens=5, prompt_lens=lens)
    for b, n in enumerate(lens):
        alone = L.greedy_generate(ids[b:b + 1, :n], params(m), max_new_tokens=5, **_oracle_kw(m))
        assert torch.equal(rag[b, 9:].cpu(), alone[0, n:]), f"sequence {b}"


def test_generate_bf16_graph_equals_eager_and_stops_on_eos():
    m = _dense(torch.bfloat16)
    ids = torch.randint(0, 1000, (4, 12), generator=torch.Generator().manual_seed(20))
    a = m.generate(ids.to(DEV), max_new_tokens=8)
    b = m.generate(ids.to(DEV), max_new_tokens=8, use_graph=False)
    assert torch.equal(a, b), "graph replays must reproduce the eager steps"
    one = m.generate(ids[:1].to(DEV), max_new_tokens=8)
    j = next(i for i in range(13, 20) if int(one[0, i]) not in one[0, 12:i].tolist())  # a token not seen before
    stop = m.generate(ids[:1].to(DEV), max_new_tokens=8, eos_token_id=int(one[0, j]))
    assert stop.shape[1] == j + 1 and torch.equal(stop, one[:, :j + 1])


def test_moe_model_forward_fp32():
    t = MoETextConfig(**_text_cfg(), num_experts=8, num_experts_per_tok=2, moe_intermediate_size=128,
                      decoder_sparse_step=1, mlp_only_layers=[1])
    vc = VisionConfig(hidden_size=128, num_layers=1, num_heads=2, intermediate_size=256, patch_size=8,
                      num_position_embeddings=64, out_hidden_size=256, deepstack_layers=())
    m = CudaQwen3VLMoeModel(Qwen3VLConfig(family="moe", vision=vc, text=t)).to(DEV, torch.float32)
    W.init_normal_(m, seed=21, include_bias=True)
    ids = torch.randint(0, 1000, (2, 30), generator=torch.Generator().manual_seed(22))
    logits, router = m(ids.to(DEV))
    assert len(router) == 1 and router[0].shape == (60, 8)  # layer 0 is MoE, layer 1 dense
    p = params(m)
    ref, _ = L.text_model(p["embed_tokens.weight"][ids], p, positions=torch.arange(30).view(1, 1, 30).expand(3, 2, 30),
                          use_moe=lambda i: i == 0, top_k=2, **_oracle_kw(m))
    assert_close(logits, ref, atol=5e-4, what="MoE model logits fp32")
