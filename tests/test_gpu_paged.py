"""GPU parity of the paged KV cache: the decode kernel and the fused q/k norm + mRoPE append
reading and writing pages through a block table, the attention module's paged path and the
greedy loop over paged caches.

A paged cache holds the same rows as a contiguous one, only placed in shuffled pages, and
the kernels run the same per-unit arithmetic on them, so every paged result must equal the
contiguous result bit for bit; the decode outputs are also checked against the fp32 oracle
at the bf16 tolerance. Page ids outside the pool (an unassigned -1 entry, an id past the
pool) are caught by the kernels' own checks: such pages read as zero rows and drop writes,
and the status word gets bit 1.
"""
import math

import pytest
import torch

from oracle import ops as O
from qwen3_5_vl_cuda_custom_amd import _lib
from qwen3_5_vl_cuda_custom_amd import kernels as K
from qwen3_5_vl_cuda_custom_amd import workloads as W
from qwen3_5_vl_cuda_custom_amd.configs import Qwen3VLConfig, TextConfig, VisionConfig
from qwen3_5_vl_cuda_custom_amd.models import CudaQwen3VLDenseModel
from qwen3_5_vl_cuda_custom_amd.modules import PagedKVCache, StaticKVCache
from tests.parity import assert_bf16_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
D = 128


def rnd(*shape, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def paginate(kc, vc, rows, P, max_pages, seed, spare=3):
    """Pools (num_pages, Hkv, P, D) holding rows [0, rows[b]) of each (B, Hkv, cap, D) cache in
    shuffled pages (unassigned pages and rows hold unrelated values), and the (B, max_pages)
    block table (-1 past a sequence's pages)."""
    B, Hkv, cap, _ = kc.shape
    need = [math.ceil(r / P) for r in rows]
    n = sum(need) + spare
    perm = torch.randperm(n, generator=torch.Generator().manual_seed(seed)).tolist()
    kp, vp = rnd(n, Hkv, P, D, seed=seed + 1), rnd(n, Hkv, P, D, seed=seed + 2)
    table = torch.full((B, max_pages), -1, dtype=torch.int32)
    i = 0
    for b in range(B):
        for j in range(need[b]):
            pg = perm[i]
            i += 1
            table[b, j] = pg
            r0, r1 = j * P, min((j + 1) * P, cap)
            kp[pg, :, :r1 - r0] = kc[b, :, r0:r1]
            vp[pg, :, :r1 - r0] = vc[b, :, r0:r1]
    return kp, vp, table


@pytest.mark.parametrize("groups,P", [(1, 32), (4, 32), (8, 64), (16, 96)])
def test_paged_decode_equals_contiguous(groups, P):
    B, Hkv, cap = 7, 2, 1120
    lens = torch.tensor([1, 31, 0, 32, 33, 257, 1100], dtype=torch.int32)
    q = rnd(B, Hkv * groups, D, seed=1)
    kc, vc = rnd(B, Hkv, cap, D, seed=2), rnd(B, Hkv, cap, D, seed=3)
    kp, vp, table = paginate(kc, vc, lens.tolist(), P, cap // P + 1, seed=4)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    dense = K.decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV), D ** -0.5)
    paged = K.decode_attention_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), lens.to(DEV), D ** -0.5,
                                     status=status)
    assert int(status.item()) == 0
    assert torch.equal(paged, dense), "paged decode must equal the contiguous decode bit for bit"
    ref = O.decode_attention(q.float()[:, :, None], kc.float(), vc.float(), lens, D ** -0.5, groups)[:, :, 0]
    assert_bf16_close(paged, ref, what=f"paged decode groups={groups} P={P}")


def test_paged_decode_append_step_advances_lengths():
    B, Hkv, G, cap, P = 5, 2, 4, 320, 32
    lens = torch.tensor([0, 3, 63, 64, 300], dtype=torch.int32)
    q = rnd(B, Hkv * G, D, seed=5)
    kc, vc = rnd(B, Hkv, cap, D, seed=6), rnd(B, Hkv, cap, D, seed=7)
    kp, vp, table = paginate(kc, vc, (lens + 1).tolist(), P, cap // P, seed=8)
    ld, lp = lens.to(DEV), lens.to(DEV)
    dense = K.decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), ld, D ** -0.5, append=True)
    paged = K.decode_attention_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), lp, D ** -0.5, append=True)
    assert torch.equal(lp.cpu(), lens + 1) and torch.equal(ld, lp)
    assert torch.equal(paged, dense)


def test_paged_decode_c3_shape():
    """The C3 decode shape (32 sequences x 8 KV heads x 4 groups, lengths U[1024, 8192]) in
    32-row pages: equal to the contiguous decode."""
    B, Hkv, G, cap, P = 32, 8, 4, 8192, 32
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(1024, 8192, (B,), generator=g, dtype=torch.int32)
    gd = torch.Generator(device=DEV).manual_seed(1)
    kc = torch.randn(B, Hkv, cap, D, generator=gd, device=DEV).to(torch.bfloat16)
    vc = torch.randn(B, Hkv, cap, D, generator=gd, device=DEV).to(torch.bfloat16)
    q = torch.randn(B, Hkv * G, D, generator=gd, device=DEV).to(torch.bfloat16)
    # every sequence's pages, shuffled over one pool (built on the device: no host copy of the cache)
    need = [math.ceil(int(n) / P) for n in lens]
    perm = torch.randperm(sum(need), generator=g)
    table = torch.full((B, cap // P), -1, dtype=torch.int32)
    kp = torch.empty(sum(need), Hkv, P, D, dtype=torch.bfloat16, device=DEV)
    vp = torch.empty_like(kp)
    i = 0
    for b in range(B):
        ids = perm[i:i + need[b]]
        i += need[b]
        table[b, :need[b]] = ids.to(torch.int32)
        ids = ids.to(DEV)
        kp[ids] = kc[b, :, :need[b] * P].reshape(Hkv, need[b], P, D).transpose(0, 1)
        vp[ids] = vc[b, :, :need[b] * P].reshape(Hkv, need[b], P, D).transpose(0, 1)
    dense = K.decode_attention(q, kc, vc, lens.to(DEV), D ** -0.5)
    paged = K.decode_attention_paged(q, kp, vp, table.to(DEV), lens.to(DEV), D ** -0.5)
    assert torch.equal(paged, dense)


def test_qk_norm_rope_paged_equals_contiguous():
    """A prefill chunk's rotated k/v rows appended at ragged offsets: the paged append writes the
    rows the contiguous append writes, and leaves every other page row untouched."""
    B, S, Hq, Hkv, P, max_pages = 3, 40, 8, 2, 32, 5
    cap = P * max_pages
    section = [24, 20, 20]
    offs = torch.tensor([0, 17, 70], dtype=torch.int32)
    q, k, v = rnd(B, S, Hq, D, seed=10), rnd(B, S, Hkv, D, seed=11), rnd(B, S, Hkv, D, seed=12)
    qw, kw = rnd(D, seed=13) * 0.1 + 1, rnd(D, seed=14) * 0.1 + 1
    pos = (offs.view(1, B, 1) + torch.arange(S).view(1, 1, S)).expand(3, B, S).to(torch.int32).contiguous()
    inv = O.mrope_inv_freq(D, 5e6).to(DEV)
    args = [t.to(DEV) for t in (q, k, v)]
    # contiguous append into (B, cap, Hkv, D) views of (B, Hkv, cap, D) caches
    kc = torch.zeros(B, Hkv, cap, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    qo_dense = torch.empty(B, S, Hq, D, dtype=torch.bfloat16, device=DEV)
    K.qk_norm_rope(*args, qo_dense, kc.transpose(1, 2), vc.transpose(1, 2), qw.to(DEV), kw.to(DEV), pos.to(DEV), inv,
                   section, 1e-6, dst_seq_offset=offs.to(DEV), dst_seq_cap=cap)
    # paged append: shuffled pages, the pools prefilled with a sentinel
    zeros = torch.zeros(B, Hkv, cap, D, dtype=torch.bfloat16)
    _, _, table = paginate(zeros, zeros, (offs + S).tolist(), P, max_pages, seed=15)
    n = int(table.max()) + 2
    kp = torch.full((n, Hkv, P, D), 7.0, dtype=torch.bfloat16, device=DEV)
    vp = torch.full_like(kp, 7.0)
    qo = torch.empty_like(qo_dense)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    K.qk_norm_rope_paged(*args, qo, kp, vp, qw.to(DEV), kw.to(DEV), pos.to(DEV), inv, section, 1e-6, table.to(DEV),
                         offs.to(DEV), status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert torch.equal(qo, qo_dense)
    written = torch.zeros(n, P, dtype=torch.bool)
    for b in range(B):
        for r in range(int(offs[b]), int(offs[b]) + S):
            pg, row = int(table[b, r // P]), r % P
            written[pg, row] = True
            assert torch.equal(kp[pg, :, row], kc[b, :, r]) and torch.equal(vp[pg, :, row], vc[b, :, r]), (b, r)
    untouched = ~written.to(DEV)
    assert bool((kp.transpose(1, 2)[untouched] == 7.0).all()) and bool((vp.transpose(1, 2)[untouched] == 7.0).all())


def test_paged_bad_page_ids_read_zero_and_set_status():
    """Page ids the kernels' own checks reject (an id past the pool, an unassigned -1): the
    decode reads those rows as zeros and the append drops them; both set status bit 1."""
    B, Hkv, G, P = 2, 2, 4, 32
    lens = torch.tensor([40, 10], dtype=torch.int32)
    q = rnd(B, Hkv * G, D, seed=20)
    kp, vp = rnd(3, Hkv, P, D, seed=21), rnd(3, Hkv, P, D, seed=22)
    table = torch.tensor([[1, 3], [-1, -1]], dtype=torch.int32)  # page 3 is past the 3-page pool
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    o = K.decode_attention_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), lens.to(DEV), D ** -0.5,
                                 status=status)
    assert int(status.item()) == _lib.STATUS_BAD_PAGE
    # the oracle over the rows as read: sequence 0's first page, then zeros
    kz = torch.zeros(B, Hkv, 64, D)
    vz = torch.zeros(B, Hkv, 64, D)
    kz[0, :, :P], vz[0, :, :P] = kp[1].float(), vp[1].float()
    ref = O.decode_attention(q.float()[:, :, None], kz, vz, lens, D ** -0.5, G)[:, :, 0]
    assert_bf16_close(o, ref, what="decode over rejected pages")
    assert bool((o[1] == 0).all())
    # append of 4 rows at rows 30..33 of sequence 0 (pages 1 and 3) and 10..13 of sequence 1 (-1)
    S = 4
    qi, ki, vi = rnd(B, S, Hkv * G, D, seed=23), rnd(B, S, Hkv, D, seed=24), rnd(B, S, Hkv, D, seed=25)
    pos = torch.zeros(3, B, S, dtype=torch.int32)
    offs = torch.tensor([30, 10], dtype=torch.int32)
    kd, vd = kp.to(DEV), vp.to(DEV)
    status.zero_()
    K.qk_norm_rope_paged(qi.to(DEV), ki.to(DEV), vi.to(DEV), torch.empty_like(qi, device=DEV), kd, vd, None, None,
                         pos.to(DEV), O.mrope_inv_freq(D, 5e6).to(DEV), [24, 20, 20], 1e-6, table.to(DEV),
                         offs.to(DEV), status=status)
    assert int(status.item()) == _lib.STATUS_BAD_PAGE
    kd, vd = kd.cpu(), vd.cpu()
    assert torch.equal(kd[1, :, :30], kp[1, :, :30]) and torch.equal(kd[0], kp[0]) and torch.equal(kd[2], kp[2])
    assert torch.equal(vd[1, :, 30:], vi[0, :2].transpose(0, 1)), "rows 30, 31 land in page 1 (no norm on v)"


def _layer_cfg():
    return W.TextLayerConfig(hidden=1024, heads=8, kv_heads=2, head_dim=D, intermediate=2048)


def _pos(starts, seq):
    p = torch.tensor(starts).view(-1, 1) + torch.arange(seq).view(1, -1)
    return p.unsqueeze(0).expand(3, -1, -1).contiguous().to(DEV)


def test_layer_paged_cache_equals_static_cache():
    """Chunked prefill with ragged lengths between the chunks, then two decode steps, through a
    PagedKVCache and a StaticKVCache: the same outputs and cache rows, bit for bit."""
    cfg = _layer_cfg()
    layer = W.make_text_layer(cfg, torch.bfloat16, DEV, seed=30)
    rope = W.make_rope(cfg, DEV)
    B, S1, S2, keep, cap = 2, 100, 60, 57, 256
    g = torch.Generator(device=DEV).manual_seed(31)
    xs = torch.randn(B, S1 + S2 + 2, cfg.hidden, generator=g, device=DEV).to(torch.bfloat16)
    static = StaticKVCache(B, cfg.kv_heads, cap, D, dtype=torch.bfloat16, device=DEV)
    paged = PagedKVCache(B, cfg.kv_heads, D, num_pages=20, max_pages=cap // 32, page_rows=32, device=DEV)
    outs = {}
    for name, cache in (("static", static), ("paged", paged)):
        ys = [layer(xs[:, :S1], rope.bind(_pos([0, 0], S1)), kv_cache=cache)[0]]
        cache.set_lens([S1, keep])
        ys.append(layer(xs[:, S1:S1 + S2], rope.bind(_pos([S1, keep], S2)), kv_cache=cache)[0])
        for t in range(2):
            ys.append(layer(xs[:, S1 + S2 + t:S1 + S2 + t + 1], rope.bind(_pos([S1 + S2 + t, keep + S2 + t], 1)),
                            kv_cache=cache)[0])
        outs[name] = ys
    assert paged.lens.cpu().tolist() == static.lens.cpu().tolist() == [S1 + S2 + 2, keep + S2 + 2]
    for i, (a, b) in enumerate(zip(outs["static"], outs["paged"])):
        assert torch.equal(a, b), f"step {i}"
    kg, vg = paged.gather(paged.max_len)
    for b, n in enumerate(paged.lens.cpu().tolist()):
        assert torch.equal(kg[b, :, :n], static.k[b, :, :n]) and torch.equal(vg[b, :, :n], static.v[b, :, :n])
    assert paged.num_free_pages == 20 - 6 - 4  # 162 and 119 rows (sequence 1 keeps its first chunk's 4 pages)


def _dense_d128(seed=40):
    vc = VisionConfig(hidden_size=128, num_layers=1, num_heads=2, intermediate_size=256, patch_size=8,
                      num_position_embeddings=64, out_hidden_size=256, deepstack_layers=(0,))
    t = TextConfig(hidden_size=256, intermediate_size=512, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=D,
                   vocab_size=1000, rope_theta=1e4, mrope_section=[24, 20, 20])
    m = CudaQwen3VLDenseModel(Qwen3VLConfig(family="dense", vision=vc, text=t)).to(DEV, torch.bfloat16)
    W.init_normal_(m, seed=seed, include_bias=True)
    with torch.no_grad():
        m.embed_tokens.weight.normal_(0, 1.0, generator=torch.Generator(device=DEV).manual_seed(seed + 1))
    return m.eval().requires_grad_(False)


def test_generate_paged_equals_static():
    """The greedy loop over paged caches (HIP-graph replays crossing page boundaries, each
    new page assigned on the host before its replay) gives the static-cache tokens."""
    m = _dense_d128()
    ids = torch.randint(0, 1000, (3, 29), generator=torch.Generator().manual_seed(41)).to(DEV)
    lens = [29, 3, 17]
    a = m.generate(ids, max_new_tokens=40, prompt_lens=lens)
    b = m.generate(ids, max_new_tokens=40, prompt_lens=lens, page_rows=32)
    c = m.generate(ids, max_new_tokens=40, prompt_lens=lens, page_rows=64, use_graph=False)
    assert torch.equal(a, b) and torch.equal(a, c)


@pytest.mark.parametrize("groups,P,Sq", [(4, 32, 77), (8, 64, 200), (4, 96, 33), (2, 32, 50), (1, 64, 90)])
def test_paged_prefill_chunk_equals_contiguous(groups, P, Sq):
    """A prefill chunk over a paged cache (read in place through the block table) returns the
    contiguous cache's result bit for bit, and advances the lengths the same way."""
    B, Hkv, cap = 5, 2, 1120
    lens = torch.tensor([0, 5, 300, 640, cap - Sq], dtype=torch.int32)
    kc, vc = rnd(B, Hkv, cap, D, seed=400), rnd(B, Hkv, cap, D, seed=401)
    q = rnd(B, Hkv * groups, Sq, D, seed=402)
    rows = (lens + Sq).tolist()
    kp, vp, table = paginate(kc, vc, rows, P, math.ceil(cap / P), seed=403)
    dl, pl = lens.to(DEV), lens.to(DEV)
    ref = K.flash_attention_cache(q.to(DEV), kc.to(DEV), vc.to(DEV), dl, D ** -0.5, groups, advance=True)
    st = torch.zeros(1, dtype=torch.int32, device=DEV)
    got = K.flash_attention_cache_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), pl, D ** -0.5, groups,
                                        advance=True, status=st)
    assert torch.equal(got, ref), "paged prefill must equal the contiguous kernel bit for bit"
    assert torch.equal(pl.cpu(), lens + Sq) and torch.equal(dl.cpu(), lens + Sq)
    assert int(st.item()) == 0
    chk = O.chunk_attention(q.float(), kc.float(), vc.float(), lens.tolist(), D ** -0.5, groups)
    assert_bf16_close(got, chk, what=f"paged chunk groups={groups} P={P}")


def test_paged_prefill_bad_page_reads_zeros_and_sets_status():
    B, Hkv, groups, P, Sq = 2, 2, 4, 32, 40
    cap = 256
    lens = torch.tensor([100, 60], dtype=torch.int32)
    kc, vc = rnd(B, Hkv, cap, D, seed=410), rnd(B, Hkv, cap, D, seed=411)
    q = rnd(B, Hkv * groups, Sq, D, seed=412)
    kp, vp, table = paginate(kc, vc, (lens + Sq).tolist(), P, cap // P, seed=413)
    table[0, 1] = 10_000  # past the pool: rows [32, 64) of sequence 0 read as zeros
    kz, vz = kc.clone(), vc.clone()
    kz[0, :, 32:64] = 0
    vz[0, :, 32:64] = 0
    st = torch.zeros(1, dtype=torch.int32, device=DEV)
    got = K.flash_attention_cache_paged(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), lens.to(DEV), D ** -0.5,
                                        groups, status=st)
    ref = K.flash_attention_cache(q.to(DEV), kz.to(DEV), vz.to(DEV), lens.to(DEV), D ** -0.5, groups)
    assert torch.equal(got, ref)
    assert int(st.item()) & _lib.STATUS_BAD_PAGE
