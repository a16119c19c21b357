"""Host-side logic that needs no GPU: KV-cache length accounting, the paged cache's page
allocator and block table, and mRoPE position checks."""
import pytest
import torch

from qwen3_5_vl_cuda_custom_amd.modules import PagedKVCache, StaticKVCache, TextMRoPE


def test_kv_cache_accounts_appends_and_refuses_overflow():
    c = StaticKVCache(2, 1, 10, 4, dtype=torch.float32, device="cpu")
    assert c.empty and c.max_len == 0
    c.reserve(8)
    assert not c.empty and (c.min_len, c.max_len) == (8, 8)
    with pytest.raises(ValueError, match="overflow"):
        c.reserve(3)
    assert c.max_len == 8  # a refused append changes nothing
    c.set_lens([3, 7])
    assert (c.min_len, c.max_len) == (3, 7) and c.lens.tolist() == [3, 7]
    c.reserve(3)
    with pytest.raises(ValueError, match="overflow"):
        c.reserve(1)
    with pytest.raises(ValueError):
        c.set_lens([3, 11])  # beyond the capacity
    with pytest.raises(ValueError):
        c.set_lens([1, 2, 3])  # wrong batch


def test_kv_cache_initial_lengths():
    c = StaticKVCache(3, 2, 16, 8, dtype=torch.float32, device="cpu", lens=torch.tensor([0, 5, 16]))
    assert (c.min_len, c.max_len) == (0, 16) and c.lens.dtype == torch.int32
    with pytest.raises(ValueError):
        c.reserve(1)


def test_paged_cache_assigns_pages_as_sequences_grow():
    c = PagedKVCache(3, 2, 8, num_pages=10, max_pages=4, page_rows=32, dtype=torch.float32, device="cpu")
    assert c.capacity == 128 and c.empty and c.num_free_pages == 10
    assert bool((c.block_table == -1).all())
    c.set_lens([5, 40, 0])  # 1, 2 and 0 pages, handed out from page 0 up
    assert c.block_table.tolist() == [[0, -1, -1, -1], [1, 2, -1, -1], [-1] * 4]
    assert c.lens.tolist() == [5, 40, 0] and (c.min_len, c.max_len) == (0, 40) and c.num_free_pages == 7
    c.reserve(30)  # 35, 70, 30 rows: one more page each
    assert c.block_table[:, :3].tolist() == [[0, 3, -1], [1, 2, 4], [5, -1, -1]] and c.num_free_pages == 4
    assert c.lens.tolist() == [5, 40, 0], "device lengths advance in the kernels, not here"
    c.release(1)
    assert c.block_table[1].tolist() == [-1] * 4 and c.lens[1] == 0 and c.num_free_pages == 7
    assert (c.min_len, c.max_len) == (0, 35)
    c.reserve(1)  # sequence 1 restarts with a recycled page (the most recently freed first)
    assert c.block_table[1, 0].item() == 1


def test_paged_cache_refuses_overflow_without_changing_state():
    c = PagedKVCache(2, 1, 4, num_pages=5, max_pages=3, page_rows=32, dtype=torch.float32, device="cpu")
    c.reserve(64)  # 2 pages each: 1 free
    table = c.block_table.clone()
    with pytest.raises(ValueError, match="pages needed"):
        c.reserve(1)  # 2 more pages, 1 free
    with pytest.raises(ValueError, match="pages needed"):
        c.check_reserve(1)
    with pytest.raises(ValueError, match="overflow"):
        c.check_reserve(33)  # 97 rows > 3 pages of 32
    assert c.host_state() == [64, 64] and torch.equal(c.block_table, table) and c.num_free_pages == 1
    c.set_lens([64, 0])
    c.prepare_append(1)  # the next append's rows get their pages now
    assert c.host_state() == [64, 0] and c.block_table[:, 2].tolist() == [4, -1] and c.num_free_pages == 0
    with pytest.raises(ValueError):
        c.set_lens([97, 0])
    with pytest.raises(ValueError):
        PagedKVCache(1, 1, 4, num_pages=2, max_pages=2, page_rows=48, device="cpu")  # not a multiple of 32


def test_paged_cache_gather_puts_pages_in_row_order():
    c = PagedKVCache(2, 2, 4, num_pages=6, max_pages=3, page_rows=32, dtype=torch.float32, device="cpu")
    c.set_lens([70, 33])  # sequence 0: pages 0, 1, 2; sequence 1: pages 3, 4
    for pg in range(6):
        c.k_pages[pg] = pg
        c.v_pages[pg] = -pg
    k, v = c.gather(70)
    assert k.shape == (2, 2, 96, 4)
    assert k[0, :, ::32, 0].tolist() == [[0, 1, 2], [0, 1, 2]]
    assert k[1, 1, ::32, 0].tolist() == [3, 4, 0]  # past its pages: page 0's rows (never attended)
    assert torch.equal(v[0], -k[0])


def test_mrope_positions_checked_and_broadcast():
    rope = TextMRoPE(128, theta=5e6, mrope_section=[24, 20, 20])
    pos = torch.arange(6).view(1, 1, 6).expand(3, 1, 6)
    b = rope.bind(pos)
    p = b.positions_int32(torch.device("cpu"), batch=2, seq=6)
    assert p.shape == (3, 2, 6) and p.dtype == torch.int32 and p.is_contiguous()
    assert torch.equal(p[:, 0], p[:, 1])
    with pytest.raises(ValueError):
        b.positions_int32(torch.device("cpu"), batch=2, seq=5)  # sequence length mismatch
    bad = rope.bind(torch.zeros(3, 3, 6, dtype=torch.int64))
    with pytest.raises(ValueError):
        bad.positions_int32(torch.device("cpu"), batch=2, seq=6)  # batch 3 for 2 sequences
    with pytest.raises(ValueError):
        rope.bind(torch.zeros(2, 1, 6)).positions_int32(torch.device("cpu"), batch=1, seq=6)  # not 3 axes
    # an int32 (3, B, S) tensor is used as is (in-place updates reach the kernels)
    own = torch.zeros(3, 2, 1, dtype=torch.int32)
    assert rope.bind(own).positions_int32(torch.device("cpu"), batch=2, seq=1).data_ptr() == own.data_ptr()


def test_paged_cache_refuses_shapes_the_paged_kernels_do_not_take():
    ok = PagedKVCache(2, 2, 128, num_pages=4, max_pages=2, page_rows=32, device="cpu")
    ok.check_kernels(4)
    ok.check_kernels(32)
    for cache, groups in ((ok, 33),
                          (PagedKVCache(2, 2, 64, num_pages=4, max_pages=2, page_rows=32, device="cpu"), 4),
                          (PagedKVCache(2, 2, 128, num_pages=4, max_pages=2, page_rows=32, dtype=torch.float32,
                                        device="cpu"), 4)):
        before = (cache.host_state(), cache.block_table.clone(), cache.num_free_pages)
        with pytest.raises(ValueError, match="paged kernels"):
            cache.check_kernels(groups)
        assert (cache.host_state(), cache.num_free_pages) == (before[0], before[2])
        assert torch.equal(cache.block_table, before[1])
