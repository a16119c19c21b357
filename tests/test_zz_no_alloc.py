"""The allocation-free decode step (q3_decode_attention_step_noalloc) through the C-ABI,
against the workspace entry point it shares its kernels with (q3_decode_attention_step):
two calls in a row, the second with a smaller batch and shorter caches."""
import pytest
import torch

from qwen3_5_vl_cuda_custom_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _strides(q, kc, vc, o):
    return _lib.i64s(q.stride(0), q.stride(1), kc.stride(0), kc.stride(1), kc.stride(2), vc.stride(0), vc.stride(1),
                     vc.stride(2), o.stride(0), o.stride(1))


def _step(name, q, kc, vc, lens, o, scale):
    B, Hq, D = q.shape
    Hkv, cap = kc.shape[1], kc.shape[2]
    args = [q.data_ptr(), kc.data_ptr(), vc.data_ptr(), lens.data_ptr(), o.data_ptr(), B, Hq, Hkv, D, cap,
            _strides(q, kc, vc, o), scale, _lib.Q3_BF16]
    if name == "q3_decode_attention_step":
        nbytes = _lib.lib().q3_decode_attention_workspace_bytes(B, Hq, Hkv, cap, D)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        args += [ws.data_ptr(), nbytes]
    _lib.call(name, *args, _lib.stream())


@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (64, 2)])
def test_noalloc_decode_step_matches_workspace_entry_point(Hq, Hkv):
    D, cap = 128, 8300
    g = torch.Generator().manual_seed(7)
    for B, lo, hi in [(32, 1024, 8192), (5, 1, 700)]:  # second call: smaller input
        lens0 = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
        q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
        kc = torch.randn(B, Hkv, cap, D, generator=g).to(torch.bfloat16).to(DEV)
        vc = torch.randn(B, Hkv, cap, D, generator=g).to(torch.bfloat16).to(DEV)
        scale = D ** -0.5
        lens_a, lens_b = lens0.to(DEV), lens0.to(DEV)
        o_a = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=DEV)
        o_b = torch.full((B, Hq, D), float("nan"), dtype=torch.bfloat16, device=DEV)
        _step("q3_decode_attention_step", q, kc, vc, lens_a, o_a, scale)
        _step("q3_decode_attention_step_noalloc", q, kc, vc, lens_b, o_b, scale)
        torch.cuda.synchronize()
        assert torch.equal(o_a, o_b), f"B={B}: outputs differ"
        assert torch.equal(lens_a.cpu(), lens0 + 1) and torch.equal(lens_b.cpu(), lens0 + 1)


def test_noalloc_refuses_requests_beyond_the_scratch():
    cap = _lib.lib().q3_decode_attention_step_noalloc_max_bytes()
    assert cap == 32 << 20
    # 1024 sequences x 32 KV heads of 32-query groups: a workspace far above the array
    need = _lib.lib().q3_decode_attention_workspace_bytes(1024, 1024, 32, 64, 128)
    assert need > cap
    q = torch.empty(1, 1, 128, dtype=torch.bfloat16, device=DEV)  # never read: refused on the host
    st = _lib.i64s(*([128] * 10))
    rc = _lib.lib().q3_decode_attention_step_noalloc(q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(),
                                                     q.data_ptr(), 1024, 1024, 32, 128, 64, st, 0.1, _lib.Q3_BF16,
                                                     _lib.stream())
    assert rc == -7 and "scratch" in _lib.error_string(rc)
