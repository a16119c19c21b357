"""The C-ABI library on the host (no GPU needed): it loads, exports every entry point that
include/q3vl.h declares, and rejects bad arguments with negative status codes before any
device work (the reference's TORCH_CHECK paths, e.g. csrc/flash_attention_op.cu:152)."""
import ctypes
import re
from pathlib import Path

import pytest

from qwen3_5_vl_cuda_custom_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
FAKE = 0x100000  # a non-null address that host-side validation never dereferences


def header_functions():
    text = (ROOT / "include" / "q3vl.h").read_text()
    return sorted(set(re.findall(r"\b(q3_\w+)\s*\(", text)))


def test_library_loads_and_reports_version():
    lib = _lib.lib()
    assert lib.q3_abi_version() == 2
    assert _lib.error_string(0) == "ok"
    assert "pointer" in _lib.error_string(-1)


def test_every_declared_entry_point_is_exported_and_bound():
    declared = header_functions()
    assert len(declared) >= 20
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in q3vl.h but not exported"
    assert set(declared) == set(_lib.EXPORTED), "ctypes signatures must cover exactly the header"


def test_symbols_are_c_linkage():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    for name in header_functions():
        assert re.search(rf"\bT {name}$", out, re.M), f"{name} is not an unmangled exported symbol"


L = None


@pytest.fixture(autouse=True)
def lib():
    global L
    L = _lib.lib()


def test_matmul_validation():
    assert L.q3_matmul(None, FAKE, None, None, FAKE, 4, 4, 4, 4, 4, 0, 4, 1, None, 0, None) == -1
    assert L.q3_matmul(FAKE, FAKE, None, None, FAKE, -1, 4, 4, 4, 4, 0, 4, 1, None, 0, None) == -2
    assert L.q3_matmul(FAKE, FAKE, None, None, FAKE, 4, 4, 8, 4, 8, 0, 4, 1, None, 0, None) == -2  # ldx < K
    assert L.q3_matmul(FAKE, FAKE, None, None, FAKE, 4, 4, 4, 4, 4, 0, 4, 7, None, 0, None) == -3
    # decode-shaped bf16 GEMM: the row-owned kernel (M <= 8 or K <= 16384) needs no
    # workspace; the stream-K kernel (M > 8, K > 16384) needs its split-K workspace
    assert L.q3_matmul_workspace_bytes(32, 4096, 12288, 1, 0) == 0
    # prefill-sized plain GEMMs: a split over K only where 256x256 tiles leave the GPU idle and K
    # is long (the planes follow the 16 KiB counter region)
    assert L.q3_matmul_workspace_bytes(1024, 4096, 12288, 1, 0) == (16 << 10) + 4 * 1024 * 4096 * 4
    assert L.q3_matmul_workspace_bytes(1024, 4096, 4096, 1, 0) == 0
    assert L.q3_matmul_workspace_bytes(4096, 4096, 12288, 1, 0) == 0
    assert L.q3_matmul_workspace_bytes(1024, 4096, 12288, 1, 1) == 0  # SwiGLU: never split
    assert L.q3_matmul_workspace_bytes(8, 4096, 20480, 1, 0) == 0
    ws = L.q3_matmul_workspace_bytes(32, 4096, 20480, 1, 0)
    assert ws > 0
    assert L.q3_matmul(FAKE, FAKE, None, None, FAKE, 32, 4096, 20480, 20480, 20480, 0, 4096, 1, None, 0, None) == -6
    assert L.q3_matmul_workspace_bytes(4096, 4096, 4096, 1, 0) == 0
    assert L.q3_matmul(FAKE, FAKE, None, None, FAKE, 0, 4, 4, 4, 4, 0, 4, 1, None, 0, None) == 0  # empty: no-op


def test_rmsnorm_matmul_validation():
    L = _lib.lib()
    ws3 = (ctypes.c_void_p * 3)(FAKE, FAKE, FAKE)
    ns = _lib.i64s(4096, 1024, 1024)
    seg = lambda x, nw, w, M, K, ldx, dt: L.q3_rmsnorm_matmul_segments(x, nw, 1e-6, w, None, ns, 3, FAKE, M, K, ldx, K,
                                                                      6144, dt, None)
    assert seg(FAKE, None, ws3, 32, 4096, 4096, 1) == -1                  # no norm weight
    assert seg(None, FAKE, ws3, 32, 4096, 4096, 1) == -1
    assert seg(FAKE, FAKE, ws3, 32, 4096, 4000, 1) == -2                  # ldx < K
    assert seg(FAKE, FAKE, ws3, 33, 4096, 4096, 1) == -5                  # prefill rows: not fused
    assert seg(FAKE, FAKE, ws3, 32, 4096, 4096, 0) == -3                  # fp32
    assert seg(FAKE, FAKE, ws3, 0, 4096, 4096, 1) == 0                    # empty: no-op
    assert seg(FAKE, FAKE + 8, ws3, 32, 4096, 4096, 1) == -4              # misaligned norm weight
    assert L.q3_rmsnorm_matmul_segments(FAKE, FAKE, 1e-6, ws3, None, ns, 5, FAKE, 32, 4096, 4096, 4096, 6144, 1,
                                        None) == -2                       # > 4 segments
    sw = lambda M, K, ldx, dt, nw=FAKE: L.q3_rmsnorm_matmul_swiglu(FAKE, nw, 1e-6, FAKE, FAKE, FAKE, M, 12288, K, ldx,
                                                                   K, 12288, dt, None)
    assert sw(32, 4096, 4096, 1, nw=None) == -1
    assert sw(64, 4096, 4096, 1) == -5
    assert sw(32, 4096, 4096, 0) == -3
    assert sw(32, 4100, 4104, 1) == -4                                    # K not a multiple of 8
    assert sw(0, 4096, 4096, 1) == 0
    assert L.q3_rmsnorm_matmul_swiglu(FAKE, FAKE, -1.0, FAKE, FAKE, FAKE, 32, 12288, 4096, 4096, 4096, 12288, 1,
                                      None) == -2                         # negative eps


def test_matmul_segments_validation():
    import ctypes
    ns = _lib.i64s(4096, 1024, 1024)
    ws3 = (ctypes.c_void_p * 3)(FAKE, FAKE, FAKE)
    assert L.q3_matmul_segments(FAKE, ws3, None, ns, 0, FAKE, 8, 4096, 4096, 4096, 6144, 1, None, 0, None) == -2
    assert L.q3_matmul_segments(FAKE, ws3, None, ns, 5, FAKE, 8, 4096, 4096, 4096, 6144, 1, None, 0, None) == -2
    assert L.q3_matmul_segments(FAKE, None, None, ns, 3, FAKE, 8, 4096, 4096, 4096, 6144, 1, None, 0, None) == -1
    holes = (ctypes.c_void_p * 3)(FAKE, None, FAKE)
    assert L.q3_matmul_segments(FAKE, holes, None, ns, 3, FAKE, 8, 4096, 4096, 4096, 6144, 1, None, 0, None) == -1
    assert L.q3_matmul_segments(FAKE, ws3, None, ns, 3, FAKE, 8, 4096, 4096, 4096, 6000, 1, None, 0, None) == -2
    assert L.q3_matmul_segments(FAKE, ws3, None, ns, 3, FAKE, 8, 4096, 4096, 4096, 6144, 7, None, 0, None) == -3
    assert L.q3_matmul_segments_workspace_bytes(8, ns, 3, 4096, 1) == 0  # row-owned kernel
    need = L.q3_matmul_segments_workspace_bytes(32, ns, 3, 20480, 1)
    assert need > 0
    assert L.q3_matmul_segments(FAKE, ws3, None, ns, 3, FAKE, 32, 20480, 20480, 20480, 6144, 1, None, 0, None) == -6
    assert L.q3_matmul_segments_workspace_bytes(4096, ns, 3, 4096, 1) == 0
    assert L.q3_matmul_segments(FAKE, ws3, None, ns, 3, FAKE, 0, 4096, 4096, 4096, 6144, 1, None, 0, None) == 0


def test_elementwise_and_norm_validation():
    assert L.q3_residual_add(FAKE, None, FAKE, 10, 1, None) == -1
    assert L.q3_residual_add(FAKE, FAKE, FAKE, -1, 1, None) == -2
    assert L.q3_residual_add(FAKE, FAKE, FAKE, 0, 1, None) == 0
    assert L.q3_gelu_tanh(FAKE, FAKE, 10, 9, None) == -3
    assert L.q3_rmsnorm(FAKE, FAKE, FAKE, 4, 0, 1e-6, 1, None) == -2
    assert L.q3_layernorm(None, FAKE, None, FAKE, 4, 4, 1e-6, 1, None) == -1
    assert L.q3_softmax(FAKE, FAKE, 4, 0, 1, None) == -2
    assert L.q3_topk(FAKE, FAKE, FAKE, 4, 8, 9, 1, None) == -2      # k > cols
    assert L.q3_topk(FAKE, FAKE, FAKE, 4, 4096, 8, 1, None) == -5   # cols beyond the register-resident kernel


def test_attention_validation():
    st = _lib.i64s(*([1] * 12))
    assert L.q3_flash_attention(FAKE, FAKE, FAKE, FAKE, None, 1, 6, 4, 8, 8, 64, st, 0.1, 1, 1, None) == -2  # Hq % Hkv
    assert L.q3_flash_attention(FAKE, FAKE, FAKE, FAKE, None, 1, 4, 4, 8, 8, 512, st, 0.1, 1, 1, None) == -5  # D > 256
    assert L.q3_flash_attention(FAKE, None, FAKE, FAKE, None, 1, 4, 4, 8, 8, 64, st, 0.1, 1, 1, None) == -1
    # (B=2, Hq=8, D=128) q/o; (B, Hkv=2, cap=100, D) caches
    d = _lib.i64s(8 * 128, 128, 2 * 100 * 128, 100 * 128, 128, 2 * 100 * 128, 100 * 128, 128, 8 * 128, 128)
    assert L.q3_decode_attention(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 8, 2, 128, 100, d, 0.1, 1, None, 0, None) == -6
    # one (m, l, O) record of the group's 4 heads per piece of a (sequence, KV head) pair: at most one
    # per pair plus one per boundary between the (at most 1024) waves of the grid
    # (after a 4352-byte header holding the work split)
    assert L.q3_decode_attention_workspace_bytes(32, 32, 8, 8193, 128) == 4352 + (1024 + 32 * 8) * 4 * 130 * 4
    assert L.q3_decode_attention_step(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 8, 2, 128, 100, d, 0.1, 1, None, 0, None) == -6
    assert L.q3_decode_attention_step(FAKE, FAKE, FAKE, None, FAKE, 2, 8, 2, 128, 100, d, 0.1, 1, None, 0, None) == -1
    # the allocation-free step: requests whose workspace exceeds its static array are refused on the host
    assert L.q3_decode_attention_step_noalloc_max_bytes() == 32 << 20
    big = _lib.i64s(*([128] * 10))
    assert L.q3_decode_attention_step_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE, 1024, 1024, 32, 128, 64, big, 0.1, 1,
                                              None) == -7
    assert L.q3_decode_attention_step_noalloc(FAKE, FAKE, FAKE, None, FAKE, 2, 8, 2, 128, 100, d, 0.1, 1,
                                              None) == -1
    assert L.q3_decode_attention_step_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 8, 2, 128, 100, d, 0.1, 1,
                                              None) == 0  # empty batch: no-op
    assert "scratch" in _lib.error_string(-7)
    # prefill chunk over a cache: lengths are required, and the chunk must fit the capacity
    assert L.q3_flash_attention_cache(FAKE, FAKE, FAKE, None, FAKE, 2, 8, 2, 16, 100, 128, st, 0.1, 1, 1, None) == -1
    assert L.q3_flash_attention_cache(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 8, 2, 101, 100, 128, st, 0.1, 1, 1,
                                      None) == -2
    assert L.q3_flash_attention_cache(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 6, 4, 16, 100, 128, st, 0.1, 1, 1,
                                      None) == -2  # Hq % Hkv
    assert L.q3_flash_attention_cache(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 8, 2, 16, 100, 128, st, 0.1, 1, 1,
                                      None) == 0  # empty batch: no-op
    # paged decode: (num_pages, Hkv=2, page_rows=32, D) pools, 4 pages per sequence
    pg = _lib.i64s(8 * 128, 128, 2 * 32 * 128, 32 * 128, 128, 2 * 32 * 128, 32 * 128, 128, 8 * 128, 128)
    ws = L.q3_decode_attention_workspace_bytes(2, 8, 2, 128, 128)
    assert L.q3_decode_attention_paged(FAKE, FAKE, FAKE, None, 4, 32, 10, FAKE, 0, FAKE, 2, 8, 2, 128, pg, 0.1, 1,
                                       FAKE, ws, None, None) == -1  # no block table
    assert L.q3_decode_attention_paged(FAKE, FAKE, FAKE, FAKE, 4, 48, 10, FAKE, 0, FAKE, 2, 8, 2, 128, pg, 0.1, 1,
                                       FAKE, ws, None, None) == -2  # page rows not a multiple of 32
    assert L.q3_decode_attention_paged(FAKE, FAKE, FAKE, FAKE, 4, 32, 10, FAKE, 0, FAKE, 2, 8, 2, 64, pg, 0.1, 1,
                                       FAKE, ws, None, None) == -5  # only the D = 128 bf16 kernel reads pages
    assert L.q3_decode_attention_paged(FAKE, FAKE, FAKE, FAKE, 4, 32, 10, FAKE, 0, FAKE, 2, 8, 2, 128, pg, 0.1, 0,
                                       FAKE, ws, None, None) == -5  # fp32
    assert L.q3_decode_attention_paged(FAKE, FAKE, FAKE, FAKE, 4, 32, 10, FAKE, 0, FAKE, 2, 8, 2, 128, pg, 0.1, 1,
                                       FAKE, ws - 16, None, None) == -6
    assert L.q3_decode_attention_paged(FAKE, FAKE, FAKE, FAKE, 4, 32, 10, FAKE, 0, FAKE, 0, 8, 2, 128, pg, 0.1, 1,
                                       FAKE, ws, None, None) == 0  # empty batch: no-op
    # fused q/k norm + mRoPE + attention: one fp32 rotary table row (D floats) per token
    assert L.q3_qk_norm_rope_attention_workspace_bytes(1, 4096, 128) == 4096 * 128 * 4
    sec = _lib.i64s(24, 20, 20)
    ws = 2 * 40 * 128 * 4

    def fused(Hq=8, Hkv=2, D=128, dtype=1, qw=FAKE, nws=ws, B=2, section=sec):
        return L.q3_qk_norm_rope_attention(FAKE, FAKE, FAKE, FAKE, qw, FAKE, FAKE, FAKE, B, 40, Hq, Hkv, D, section,
                                           1e-6, st, 0.1, 1, dtype, FAKE, nws, None)
    assert fused(qw=None) == -1  # the norm weights are required
    assert fused(Hq=6, Hkv=4) == -2
    assert fused(section=_lib.i64s(24, 20, 19)) == -2
    assert fused(dtype=0) == -3  # bf16 only
    assert fused(D=72, section=_lib.i64s(12, 12, 12)) == -5  # rotate-half pairs must share a lane
    assert fused(D=96, section=_lib.i64s(16, 16, 16)) == -5  # no 12-lane groups in the k kernel
    assert fused(Hq=4, Hkv=2) == -5  # GQA groups of 2: not the pipelined kernel
    assert fused(nws=ws - 4) == -6
    assert fused(B=0) == 0  # empty batch: no-op


def test_rope_validation():
    s3 = _lib.i64s(1, 1, 1)
    sec = _lib.i64s(24, 20, 19)  # does not sum to D_rope / 2
    assert L.q3_mrope(FAKE, FAKE, FAKE, FAKE, 1, 1, 1, 128, 128, sec, s3, s3, s3, 1, 0, None) == -2
    assert L.q3_rope(FAKE, FAKE, FAKE, FAKE, 1, 1, 1, 64, 65, s3, s3, 0, 65, 1, 0, None) == -2  # odd D_rope
    st = _lib.i64s(*([1] * 18))
    sec = _lib.i64s(24, 20, 20)
    assert L.q3_qk_norm_rope(FAKE, FAKE, None, FAKE, FAKE, None, None, None, FAKE, FAKE, None, 0, 1, 1, 1, 1, 72,
                             sec, 1e-6, st, 1, None) == -5  # head dim not a multiple of 16
    assert L.q3_qk_norm_rope(FAKE, FAKE, FAKE, FAKE, FAKE, None, None, None, FAKE, FAKE, None, 0, 1, 1, 1, 1, 128,
                             sec, 1e-6, st, 1, None) == -1  # v_in without v_out
    assert L.q3_qk_norm_rope_paged(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, None, 4, 32, 10, FAKE,
                                   1, 1, 1, 1, 128, sec, 1e-6, st, 1, None, None) == -1  # no block table
    assert L.q3_qk_norm_rope_paged(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, FAKE, 4, 32, 10, None,
                                   1, 1, 1, 1, 128, sec, 1e-6, st, 1, None, None) == -1  # no lengths
    assert L.q3_qk_norm_rope_paged(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, FAKE, 4, 40, 10, FAKE,
                                   1, 1, 1, 1, 128, sec, 1e-6, st, 1, None, None) == -2  # page rows


def test_moe_validation():
    assert L.q3_moe_route(FAKE, FAKE, FAKE, None, 16, 8, 9, 1, None) == -2           # k > E
    assert L.q3_moe_route(FAKE, FAKE, FAKE, None, 16, 1024, 8, 1, None) == -5        # E beyond register-resident
    # router with the split-K logits GEMM: 4096 x 2048 x 128 takes 8 splits of 256 columns
    assert L.q3_moe_router_workspace_bytes(4096, 2048, 128) == 8 * 4096 * 128 * 4
    assert L.q3_moe_router_workspace_bytes(77, 520, 96) == 77 * 96 * 4  # 520 has no 64-column split
    assert L.q3_moe_router(FAKE, FAKE, FAKE, FAKE, FAKE, None, 16, 64, 8, 2, 1, None, 0, None) == -6
    assert L.q3_moe_router(FAKE, FAKE, FAKE, FAKE, FAKE, None, 16, 60, 8, 2, 1, FAKE, 1 << 20, None) == -4  # H % 8
    assert L.q3_moe_router(FAKE, None, FAKE, FAKE, FAKE, None, 16, 64, 8, 2, 1, FAKE, 1 << 20, None) == -1
    assert L.q3_moe_router(FAKE, FAKE, FAKE, FAKE, FAKE, None, 16, 64, 8, 9, 1, FAKE, 1 << 20, None) == -2  # k > E
    assert L.q3_moe_router(FAKE, FAKE, FAKE, FAKE, FAKE, None, 0, 64, 8, 2, 1, None, 0, None) == 0  # no tokens
    assert L.q3_moe_experts(FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, 16, 20, 8, 4, 2, None, 0, None) == -5  # H % 8
    ws = L.q3_moe_experts_workspace_bytes(4096, 2048, 768, 128, 8)
    assert ws > 4096 * 8 * (2048 + 768) * 2
    assert L.q3_moe_experts(FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, 16, 64, 32, 4, 2, None, 0, None) == -6
    assert L.q3_index_add(FAKE, FAKE, FAKE, 5, 3, 4, 1, None, 0, None, None) == -6
    assert L.q3_index_add(FAKE, None, FAKE, 5, 3, 4, 1, None, 0, None, None) == -1
    assert L.q3_index_add(FAKE, FAKE, FAKE, 0, 3, 4, 1, None, 0, None, None) == 0  # no sources: no-op
    # dispatch tables on their own
    assert L.q3_moe_permute(FAKE, FAKE, FAKE, FAKE, FAKE, None, 16, 8, 2, FAKE, 1 << 20, None) == -1
    assert L.q3_moe_permute(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 16, 8, 9, FAKE, 1 << 20, None) == -2  # k > E
    assert L.q3_moe_permute(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 16, 8, 2, None, 0, None) == -6
    assert 0 < L.q3_moe_permute_workspace_bytes(4096, 128, 8) < ws
    assert L.q3_moe_permute(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 8, 2, None, 0, None) == 0
