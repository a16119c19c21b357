"""Host-side logic that needs no GPU: KV-cache length accounting and mRoPE position checks."""
import pytest
import torch

from qwen3_5_vl_cuda_custom_amd.modules import StaticKVCache, TextMRoPE


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
