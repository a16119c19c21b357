"""Module-level parity on the BASELINE configurations (C1-C5).

The bf16 modules are compared with the fp32 oracle composition of the same
seeded weights and inputs (bf16-rounded values upcast to fp32). Large cases run
the oracle's torch code on the GPU in fp32 (it is device-agnostic); small ones
on the CPU.
"""
import pytest
import torch

from oracle import layers as L
from oracle import ops as O
from qwen3_5_vl_cuda_custom_amd import workloads as W
from qwen3_5_vl_cuda_custom_amd.modules import TextMRoPE
from tests.parity import assert_bf16_close, assert_close, assert_layer_parity, metrics

pytestmark = pytest.mark.gpu
DEV = "cuda"


def params(module, device):
    return {n: t.detach().float().to(device) for n, t in module.state_dict().items()}


def oracle_text_layer(layer, cfg, x, pos, device, past_kv=None, router_logits=None, bf16_path=False):
    """fp32 oracle of the layer; bf16_path=True rounds every op output to bf16 (the reference's bf16 path)."""
    p = params(layer, device)
    cos3, sin3 = O.mrope_cos_sin(pos.to(device), cfg.head_dim, cfg.theta)
    return L.text_decoder_layer(x.float().to(device), p, num_heads=cfg.heads, num_kv_heads=cfg.kv_heads,
                                head_dim=cfg.head_dim, eps=cfg.eps, cos_3d=cos3, sin_3d=sin3,
                                mrope_section=list(cfg.mrope_section), use_moe=cfg.use_moe, top_k=cfg.top_k,
                                past_kv=past_kv, router_logits=router_logits,
                                rd=O.round_bf16 if bf16_path else (lambda t: t))


def test_c1_tiny_layer_fp32():
    cfg = W.C1
    layer = W.make_text_layer(cfg, torch.float32, DEV, seed=0)
    x, pos = W.text_inputs(cfg, 1, 128, torch.float32, DEV, seed=0)
    rope = W.make_rope(cfg, DEV)
    y, logits, (k, v) = layer(x, rope.bind(pos))
    ref, _, (rk, rv) = oracle_text_layer(layer, cfg, x, pos, "cpu")
    assert logits is None
    assert_close(y, ref, atol=2e-4, what="C1 layer fp32")
    assert_close(k, rk, atol=2e-4, what="C1 k")
    assert_close(v, rv, atol=2e-4, what="C1 v")
    # the unfused path (any mrope callable) gives the same answer
    y2, _, _ = layer(x, lambda q, kk: rope.apply(q, kk, pos))
    assert_close(y2, ref, atol=2e-4, what="C1 layer fp32 (unfused rope callable)")


@pytest.mark.parametrize("seq", [256, 1024])
def test_c2_layer_bf16_reduced_seq(seq):
    cfg = W.C2
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV, seed=0)
    x, pos = W.text_inputs(cfg, 1, seq, torch.bfloat16, DEV, seed=0)
    y, _, (k, v) = layer(x, W.make_rope(cfg, DEV).bind(pos))
    ref, _, (rk, rv) = oracle_text_layer(layer, cfg, x, pos, DEV)
    emu, _, (ek, ev) = oracle_text_layer(layer, cfg, x, pos, DEV, bf16_path=True)
    assert_layer_parity(k, rk, ek, what=f"C2 k S={seq}")
    assert_layer_parity(v, rv, ev, what=f"C2 v S={seq}")
    assert_layer_parity(y, ref, emu, what=f"C2 layer S={seq}")


@pytest.mark.slow
def test_c2_layer_bf16_full_seq4096():
    cfg = W.C2
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV, seed=0)
    x, pos = W.text_inputs(cfg, 1, 4096, torch.bfloat16, DEV, seed=0)
    y, _, _ = layer(x, W.make_rope(cfg, DEV).bind(pos))
    ref, _, _ = oracle_text_layer(layer, cfg, x, pos, DEV)
    emu, _, _ = oracle_text_layer(layer, cfg, x, pos, DEV, bf16_path=True)
    assert_layer_parity(y, ref, emu, what="C2 layer S=4096")
    # determinism: a second run is bitwise identical
    y2, _, _ = layer(x, W.make_rope(cfg, DEV).bind(pos))
    assert torch.equal(y, y2)


@pytest.mark.slow
def test_c2_layer_bf16_full_seq16384():
    """The third C2 length: the fp32 oracle on the GPU (its attention in fp32)."""
    cfg = W.C2
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV, seed=0)
    x, pos = W.text_inputs(cfg, 1, 16384, torch.bfloat16, DEV, seed=0)
    y, _, (k, v) = layer(x, W.make_rope(cfg, DEV).bind(pos))
    ref, _, (rk, rv) = oracle_text_layer(layer, cfg, x, pos, DEV)
    emu, _, (ek, ev) = oracle_text_layer(layer, cfg, x, pos, DEV, bf16_path=True)
    assert_layer_parity(k, rk, ek, what="C2 k S=16384")
    assert_layer_parity(v, rv, ev, what="C2 v S=16384")
    del rk, rv, ek, ev
    assert_layer_parity(y, ref, emu, what="C2 layer S=16384")


def _positions(starts, seq):
    """(3, B, seq) int64 text positions starts[b] + 0..seq-1 on every axis."""
    p = torch.tensor(starts).view(-1, 1) + torch.arange(seq).view(1, -1)
    return p.unsqueeze(0).expand(3, -1, -1).contiguous().to(DEV)


@pytest.mark.parametrize("cfg", [
    W.TextLayerConfig(hidden=1024, heads=8, kv_heads=2, head_dim=128, intermediate=2048),
    W.TextLayerConfig(hidden=512, heads=8, kv_heads=4, head_dim=64, intermediate=1024, mrope_section=(12, 10, 10)),
])
def test_kv_cache_chunked_prefill_ragged_then_decode(cfg):
    """Prefill in two chunks into a StaticKVCache, with ragged lengths between them
    (sequence 1 keeps only its first 57 tokens), then one decode step. Chunked
    causal attention equals attention over the whole sequence at once, so every
    output and cache row must match the fp32 oracle's layer over each sequence's
    full token list."""
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV, seed=11)
    rope = W.make_rope(cfg, DEV)
    B, S1, S2, keep, cap = 2, 100, 60, 57, 256
    g = torch.Generator(device=DEV).manual_seed(12)
    xs = torch.randn(B, S1 + S2 + 1, cfg.hidden, generator=g, device=DEV).to(torch.bfloat16)
    cache = W.StaticKVCache(B, cfg.kv_heads, cap, cfg.head_dim, dtype=torch.bfloat16, device=DEV)
    y1, _, _ = layer(xs[:, :S1], rope.bind(_positions([0, 0], S1)), kv_cache=cache)
    cache.set_lens([S1, keep])
    y2, _, _ = layer(xs[:, S1:S1 + S2], rope.bind(_positions([S1, keep], S2)), kv_cache=cache)
    y3, _, _ = layer(xs[:, S1 + S2:], rope.bind(_positions([S1 + S2, keep + S2], 1)), kv_cache=cache)
    assert cache.lens.cpu().tolist() == [S1 + S2 + 1, keep + S2 + 1]
    seqs = [xs[0:1], torch.cat([xs[1:2, :keep], xs[1:2, S1:]], dim=1)]
    outs = [torch.cat([y1[0:1], y2[0:1], y3[0:1]], dim=1), torch.cat([y1[1:2, :keep], y2[1:2], y3[1:2]], dim=1)]
    for b in range(B):
        n = seqs[b].shape[1]
        pos = _positions([0], n)
        ref, _, (rk, rv) = oracle_text_layer(layer, cfg, seqs[b], pos, DEV)
        emu, _, (ek, ev) = oracle_text_layer(layer, cfg, seqs[b], pos, DEV, bf16_path=True)
        assert_layer_parity(outs[b], ref, emu, what=f"chunked prefill + decode, sequence {b}")
        assert_layer_parity(cache.k[b:b + 1, :, :n], rk, ek, what=f"cache k, sequence {b}")
        assert_layer_parity(cache.v[b:b + 1, :, :n], rv, ev, what=f"cache v, sequence {b}")


def test_past_kv_reference_contract():
    """The reference's cache form (modules/attention.py:89-96): past_kv=(k, v) tensors grown
    by torch.cat, attention causal only when Sq == Sk, so a one-token step attends to the
    whole cache and a multi-token step attends non-causally to everything."""
    cfg = W.TextLayerConfig(hidden=1024, heads=8, kv_heads=2, head_dim=128, intermediate=2048)
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV, seed=21)
    rope = W.make_rope(cfg, DEV)
    g = torch.Generator(device=DEV).manual_seed(22)
    x = torch.randn(1, 54, cfg.hidden, generator=g, device=DEV).to(torch.bfloat16)
    y0, _, kv0 = layer(x[:, :48], rope.bind(_positions([0], 48)))
    y1, _, kv1 = layer(x[:, 48:49], rope.bind(_positions([48], 1)), past_kv=kv0)
    y2, _, kv2 = layer(x[:, 49:], rope.bind(_positions([49], 5)), past_kv=kv1)
    assert kv1[0].shape == (1, cfg.kv_heads, 49, cfg.head_dim) and kv2[1].shape == (1, cfg.kv_heads, 54, cfg.head_dim)
    assert torch.equal(kv2[0][:, :, :48], kv0[0]), "the cache prefix is carried unchanged"
    for xs, start, past, y, kv in [(x[:, 48:49], 48, kv0, y1, kv1), (x[:, 49:], 49, kv1, y2, kv2)]:
        past32 = (past[0].float(), past[1].float())
        pos = _positions([start], xs.shape[1])
        ref, _, (rk, _) = oracle_text_layer(layer, cfg, xs, pos, DEV, past_kv=past32)
        emu, _, (ek, _) = oracle_text_layer(layer, cfg, xs, pos, DEV, past_kv=past32, bf16_path=True)
        assert_layer_parity(y, ref, emu, what=f"past_kv step of {xs.shape[1]} token(s)")
        assert_layer_parity(kv[0], rk, ek, what=f"past_kv grown k ({xs.shape[1]} token(s))")


def test_batch_one_positions_broadcast():
    """(3, 1, S) positions rotate every sequence of a batch alike (TextMRoPE.apply's
    broadcast), identical to the explicit (3, B, S) form."""
    cfg = W.TextLayerConfig(hidden=1024, heads=8, kv_heads=2, head_dim=128, intermediate=2048)
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV, seed=23)
    rope = W.make_rope(cfg, DEV)
    x, pos = W.text_inputs(cfg, 2, 40, torch.bfloat16, DEV, seed=24)
    a, _, _ = layer(x, rope.bind(pos[:, :1]))
    b, _, _ = layer(x, rope.bind(pos))
    assert torch.equal(a, b)
    with pytest.raises(ValueError):
        layer(x, rope.bind(pos[:, :, :39]))


def test_c3_decode_layer_against_per_sequence_oracle():
    cfg = W.C2
    case = W.make_decode_case(cfg, batch=32, capacity=8193, device=DEV, seed=0)
    assert int(case.lens.sum()) == 172058  # seed-0 lengths from the benchmark definition
    k0, v0 = case.cache.k.clone(), case.cache.v.clone()
    y, _, _ = case.layer(case.x, case.rope.bind(case.positions), kv_cache=case.cache)
    assert torch.equal(case.cache.lens.cpu(), (case.lens + 1).to(torch.int32))
    p = params(case.layer, DEV)
    outs, refs, emus = [], [], []
    for b in range(32):
        Lb = int(case.lens[b])
        pos = case.positions[:, b:b + 1]
        cos3, sin3 = O.mrope_cos_sin(pos, cfg.head_dim, cfg.theta)
        past = (k0[b:b + 1, :, :Lb].float(), v0[b:b + 1, :, :Lb].float())
        kw = dict(num_heads=cfg.heads, num_kv_heads=cfg.kv_heads, head_dim=cfg.head_dim, eps=cfg.eps, cos_3d=cos3,
                  sin_3d=sin3, mrope_section=list(cfg.mrope_section), past_kv=past)
        ref, _, (rk, rv) = L.text_decoder_layer(case.x[b:b + 1].float(), p, **kw)
        emu, _, _ = L.text_decoder_layer(case.x[b:b + 1].float(), p, rd=O.round_bf16, **kw)
        outs.append(y[b:b + 1])
        refs.append(ref)
        emus.append(emu)
        assert_bf16_close(case.cache.v[b:b + 1, :, Lb], rv[:, :, Lb], what=f"appended v {b}")
        if b % 8 == 0:
            assert torch.equal(case.cache.k[b, :, :Lb], k0[b, :, :Lb]), "cache rows before L_b must be untouched"
    assert_layer_parity(torch.cat(outs), torch.cat(refs), torch.cat(emus), what="C3 decode B=32")


def test_decode_step_graph_replays_match_eager():
    """Three decode tokens through a captured layer step equal three eager steps, bit for bit."""
    from qwen3_5_vl_cuda_custom_amd.modules import StepGraph
    cfg = W.TextLayerConfig(hidden=1024, heads=8, kv_heads=2, head_dim=128, intermediate=2816)
    B, cap, steps = 4, 300, 3
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV, seed=3)
    rope = W.make_rope(cfg, DEV)
    g = torch.Generator(device=DEV).manual_seed(4)
    xs = [torch.randn(B, 1, cfg.hidden, generator=g, device=DEV).to(torch.bfloat16) for _ in range(steps)]
    lens0 = torch.tensor([5, 17, 64, 200], dtype=torch.int32)

    def fresh_cache():
        c = W.StaticKVCache(B, cfg.kv_heads, cap, cfg.head_dim, dtype=torch.bfloat16, device=DEV, lens=lens0)
        gg = torch.Generator(device=DEV).manual_seed(5)
        c.k.normal_(generator=gg)
        c.v.normal_(generator=gg)
        return c

    # eager reference
    cache = fresh_cache()
    eager = []
    for t in range(steps):
        pos = (lens0 + t).to(DEV).view(1, B, 1).expand(3, B, 1).to(torch.int32).contiguous()
        y, _, _ = layer(xs[t], rope.bind(pos), kv_cache=cache)
        eager.append(y.clone())
    k_ref, v_ref = cache.k.clone(), cache.v.clone()

    # captured step: static x / positions, the cache lengths advance inside the graph
    cache = fresh_cache()
    x_in = torch.empty_like(xs[0])
    pos32 = torch.empty(3, B, 1, dtype=torch.int32, device=DEV)
    binding = rope.bind(pos32)
    lens_saved = cache.lens.clone()
    x_in.copy_(xs[0])
    pos32.copy_(lens0.to(DEV).view(1, B, 1).expand(3, B, 1))
    graph = StepGraph(lambda: layer(x_in, binding, kv_cache=cache)[0], warmup=1, caches=[cache])
    # warm-up and capture advanced the lengths and wrote rows: start over
    cache.set_lens(lens_saved)
    junk = torch.randn(1 << 20, device=DEV)
    for t in range(steps):
        x_in.copy_(xs[t])
        pos32.copy_((lens0 + t).to(DEV).view(1, B, 1).expand(3, B, 1))
        out = graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[t]), f"replay {t} differs from the eager step"
        float(junk.sum())  # eager work between replays
    assert torch.equal(cache.lens.cpu(), lens0 + steps)
    assert cache.max_len == int(lens0.max()) + steps  # replays accounted on the host
    for b in range(B):
        n = int(lens0[b]) + steps
        assert torch.equal(cache.k[b, :, :n], k_ref[b, :, :n]) and torch.equal(cache.v[b, :, :n], v_ref[b, :, :n])


def test_c4_moe_layer_reduced_tokens():
    cfg = W.C4
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV, seed=0)
    x, pos = W.text_inputs(cfg, 1, 512, torch.bfloat16, DEV, seed=0)
    y, logits, _ = layer(x, W.make_rope(cfg, DEV).bind(pos))
    assert logits.shape == (512, cfg.num_experts) and logits.dtype == torch.bfloat16
    # Route the oracle with the device's own logits: identical input, so the
    # top-k indices must agree bit-exactly.
    ref, _, _ = oracle_text_layer(layer, cfg, x, pos, DEV, router_logits=logits.float())
    emu, _, _ = oracle_text_layer(layer, cfg, x, pos, DEV, router_logits=logits.float(), bf16_path=True)
    assert_layer_parity(y, ref, emu, what="C4 MoE layer")


@pytest.mark.slow
def test_c4_moe_layer_full_tokens():
    """The benchmarked C4 size (4096 tokens, ~256 rows per expert: the 128x256 grouped
    tiles and their XCD deal), routed with the device's logits as above."""
    cfg = W.C4
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV, seed=0)
    x, pos = W.text_inputs(cfg, 1, 4096, torch.bfloat16, DEV, seed=0)
    y, logits, _ = layer(x, W.make_rope(cfg, DEV).bind(pos))
    ref, _, _ = oracle_text_layer(layer, cfg, x, pos, DEV, router_logits=logits.float())
    emu, _, _ = oracle_text_layer(layer, cfg, x, pos, DEV, router_logits=logits.float(), bf16_path=True)
    assert_layer_parity(y, ref, emu, what="C4 MoE layer T=4096")


def test_c4_router_indices_bit_exact_full():
    cfg = W.C4
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV, seed=0)
    x, _ = W.text_inputs(cfg, 1, 4096, torch.bfloat16, DEV, seed=0)
    logits, idx, w = layer.mlp.route(x.view(-1, cfg.hidden))
    probs = O.softmax(logits.float().cpu())
    rv, ri = O.topk(probs, cfg.top_k)
    assert torch.equal(idx.long().cpu(), ri)
    assert_bf16_close(w, rv / rv.sum(-1, keepdim=True), max_abs=4e-3, what="routing weights")


def test_c5_vision_block_full():
    cfg = W.C5
    blk = W.make_vision_block(cfg, torch.bfloat16, DEV, seed=0)
    pe = W.make_patch_embed(cfg, torch.bfloat16, DEV, seed=0)
    patches = W.vision_inputs(cfg, torch.bfloat16, DEV, seed=0)
    h = pe(patches)
    assert h.shape == (4 * 784, 1152)
    ref_h = L.patch_embed(patches.float(), pe.weight.float(), pe.bias.float(), 3, 2, 16)
    assert_bf16_close(h, ref_h, what="C5 patch embed")
    cos, sin = W.vision_rope_cos_sin(cfg, DEV)
    x = h.view(cfg.images, cfg.patches_per_image, cfg.hidden)
    y = blk(x, cos, sin)
    pb = params(blk, DEV)
    ref = L.vision_block(x.float(), pb, num_heads=cfg.heads, cos=cos, sin=sin, eps=cfg.eps)
    emu = L.vision_block(x.float(), pb, num_heads=cfg.heads, cos=cos, sin=sin, eps=cfg.eps, rd=O.round_bf16)
    assert_layer_parity(y, ref, emu, what="C5 vision block")


def test_vision_rope_tables_match_oracle():
    cfg = W.C5
    cos, sin = W.vision_rope_cos_sin(cfg, "cpu")
    rc, rs = L.vision_rope_tables([cfg.grid], cfg.head_dim, cfg.theta, cfg.merge)
    assert torch.allclose(cos, rc, atol=1e-6) and torch.allclose(sin, rs, atol=1e-6)


def test_modules_param_contract():
    """Parameter names and shapes equal the reference's (modules/*.py)."""
    cfg = W.C2
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV)
    shapes = {n: tuple(t.shape) for n, t in layer.state_dict().items()}
    assert shapes == {
        "input_layernorm.weight": (4096,), "post_attention_layernorm.weight": (4096,),
        "self_attn.q_proj.weight": (4096, 4096), "self_attn.k_proj.weight": (1024, 4096),
        "self_attn.v_proj.weight": (1024, 4096), "self_attn.o_proj.weight": (4096, 4096),
        "self_attn.q_norm.weight": (128,), "self_attn.k_norm.weight": (128,),
        "mlp.gate_proj.weight": (12288, 4096), "mlp.up_proj.weight": (12288, 4096),
        "mlp.down_proj.weight": (4096, 12288)}
    moe = W.make_text_layer(W.C4, torch.bfloat16, DEV)
    ms = {n: tuple(t.shape) for n, t in moe.state_dict().items() if n.startswith("mlp.")}
    assert ms == {"mlp.gate_weight": (128, 2048), "mlp.gate_up_proj": (128, 1536, 2048),
                  "mlp.down_proj": (128, 2048, 768)}
