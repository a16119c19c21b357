"""Op-level parity: each HIP kernel (through the C-ABI) against the CPU oracle on seeded inputs.

bf16 cases: the oracle runs in fp32 on the same bf16-rounded inputs; tolerance
max-abs 2e-2 / mean-rel 5e-3. fp32 cases (the reference's own test style,
tests/test_kernels.py): tight absolute tolerances. Indices: exact.
"""
import math

import pytest
import torch

from oracle import ops as O
from qwen3_5_vl_cuda_custom_amd import _lib
from qwen3_5_vl_cuda_custom_amd import kernels as K
from tests.parity import assert_bf16_close, assert_close, assert_layer_parity, assert_within_ulp, bf16_round

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rnd(*shape, seed=0, std=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def gpu(t):
    return t.to(DEV)


def f32(t):
    return t.float()


# ------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("M,N,Kd,bias", [
    (8, 32, 64, True),        # reference test shape (tests/test_kernels.py:157-162), skinny path
    (32, 4096, 4096, False),  # decode q/o projection (skinny, split-K)
    (33, 520, 264, True),     # just past the skinny bound, ragged N
    (300, 520, 264, True),    # ragged M/N, small K
    (512, 1024, 4096, False), # k/v projection shape at S=512
    (256, 1152, 4304, True),  # vision fc2: K tail (4304 = 67*64 + 16)
    (1024, 4096, 4096, False),
    (1024, 1536, 2048, False),
    (4096, 4096, 512, True),     # >= 256 tiles of 256x256: the direct-to-LDS kernel
    (4000, 4200, 520, True),     # same kernel with ragged M, N and a K tail
    (4100, 3840, 512, True),     # 256x256 tiles whose last m-tile has 4 rows: its upper waves skip their MFMAs
])
def test_matmul_bf16(M, N, Kd, bias):
    x = rnd(M, Kd, seed=1)
    w = rnd(N, Kd, seed=2, std=0.02)
    b = rnd(N, seed=3, std=0.02) if bias else None
    y = K.matmul(gpu(x), gpu(w), gpu(b) if bias else None)
    ref = O.linear(f32(x), f32(w), f32(b) if bias else None)
    assert_bf16_close(y, ref, what=f"matmul {M}x{N}x{Kd}")


def test_matmul_residual_fused():
    x, w, r = rnd(200, 512, seed=4), rnd(384, 512, seed=5, std=0.02), rnd(200, 384, seed=6)
    y = K.matmul(gpu(x), gpu(w), residual=gpu(r))
    assert_bf16_close(y, O.linear(f32(x), f32(w)) + f32(r), what="matmul+residual")
    # large: residual and bias enter the direct-to-LDS kernel's accumulators
    xl, wl, rl, bl = rnd(4096, 320, seed=60), rnd(4100, 320, seed=61, std=0.02), rnd(4096, 4100, seed=62), \
        rnd(4100, seed=63, std=0.02)
    yl = K.matmul(gpu(xl), gpu(wl), gpu(bl), residual=gpu(rl))
    assert_bf16_close(yl, O.linear(f32(xl), f32(wl), f32(bl)) + f32(rl), what="large matmul+bias+residual")
    y2 = K.matmul(gpu(x[:16]), gpu(w), residual=gpu(r[:16]))  # skinny path epilogue
    assert_bf16_close(y2, O.linear(f32(x[:16]), f32(w)) + f32(r[:16]), what="skinny matmul+residual")


@pytest.mark.parametrize("M,N,Kd,bias,res", [
    (1024, 4096, 12288, False, True),   # the S=1024 down projection: 4 splits of 3072
    (1000, 4000, 12288, True, True),    # ragged M and N, bias and residual: 4 splits
    (1024, 2048, 12288, False, False),  # 8 splits, plain store
])
def test_matmul_split_k(M, N, Kd, bias, res):
    """Few-tile, long-K GEMMs take the split over K (fp32 partial planes summed in split order,
    then bias, residual, one rounding): the plan and its workspace, and parity with the oracle."""
    ws = _lib.lib().q3_matmul_workspace_bytes(M, N, Kd, 1, 0)
    assert ws > M * N * 4, "the split plan must ask for its partial planes"
    x, w = rnd(M, Kd, seed=70), rnd(N, Kd, seed=71, std=Kd ** -0.5)
    b = rnd(N, seed=72, std=0.02) if bias else None
    r = rnd(M, N, seed=73) if res else None
    y = K.matmul(gpu(x), gpu(w), gpu(b) if bias else None, residual=gpu(r) if res else None)
    ref = O.linear(f32(x), f32(w), f32(b) if bias else None)
    if res:
        ref = ref + f32(r)
    assert_bf16_close(y, ref, what=f"split-K matmul {M}x{N}x{Kd}")
    again = K.matmul(gpu(x), gpu(w), gpu(b) if bias else None, residual=gpu(r) if res else None)
    assert torch.equal(y, again), "the split-K path must be deterministic"


@pytest.mark.parametrize("M,N,Kd,swiglu", [
    (1024, 12288, 4096, True),   # the S=1024 gate/up: 768 tiles of 128x256 on the 16x16x32 loop
    (1000, 6000, 4096, False),   # q/k/v-sized, ragged M and N: 128x256 tiles, 16x16x32 loop, bias
    (1024, 6144, 1024, False),   # K < 2048: the same tiles on the 32x32x16 loop
    (1000, 6000, 2056, False),   # the 16x16x32 loop's shortest K loops, a 8-wide last stage
    (1024, 12288, 2104, True),   # (its W ring runs two stages ahead of X: 2 X + 4 W slots)
])
def test_matmul_128x256_tiles(M, N, Kd, swiglu):
    std = Kd ** -0.5
    x = rnd(M, Kd, seed=90)
    if swiglu:
        wg, wu = rnd(N, Kd, seed=91, std=std / 2), rnd(N, Kd, seed=92, std=std / 2)
        y = K.matmul_swiglu(gpu(x), gpu(wg), gpu(wu))
        ref = O.swiglu(O.linear(f32(x), f32(wg)), O.linear(f32(x), f32(wu)))
    else:
        w, b = rnd(N, Kd, seed=91, std=std), rnd(N, seed=92, std=0.02)
        y = K.matmul(gpu(x), gpu(w), gpu(b))
        ref = O.linear(f32(x), f32(w), f32(b))
    assert_bf16_close(y, ref, what=f"128x256 tiles {M}x{N}x{Kd} swiglu={swiglu}")


@pytest.mark.parametrize("M", [7, 32, 300, 1024, 4100, 8192])
def test_matmul_swiglu(M):
    x, wg, wu = rnd(M, 1024, seed=7), rnd(1536, 1024, seed=8, std=0.02), rnd(1536, 1024, seed=9, std=0.02)
    y = K.matmul_swiglu(gpu(x), gpu(wg), gpu(wu))
    ref = O.swiglu(O.linear(f32(x), f32(wg)), O.linear(f32(x), f32(wu)))
    assert_bf16_close(y, ref, what=f"matmul_swiglu M={M}")


@pytest.mark.parametrize("M,ns,bias", [
    (600, (1024, 256, 256), False),   # tiled, one launch (starts are multiples of 256)
    (600, (512, 256, 256), True),     # tiled with per-segment bias
    (4096, (4096, 1024, 1024), True), # the q/k/v shape: 256x192 tiles straddle segment starts
    (4096, (4096, 2048), True),       # two segments, both with bias
    (2048, (1040, 512, 48), True),    # starts on 16-row (not tile) boundaries, one launch
    (300, (200, 72, 72), True),       # unaligned starts: one launch per segment
    (32, (1024, 256, 256), False),    # skinny, one launch
    (5, (96, 32, 32), True),          # skinny with bias
    (9, (100, 20), False),            # skinny, unaligned: per segment
])
def test_matmul_segments(M, ns, bias):
    Kd = 512
    x = rnd(M, Kd, seed=40)
    ws = [rnd(n, Kd, seed=41 + i, std=0.02) for i, n in enumerate(ns)]
    bs = [rnd(n, seed=50 + i, std=0.02) if bias and (i != 1 or len(ns) == 2) else None for i, n in enumerate(ns)]
    y = K.matmul_segments(gpu(x), [gpu(w) for w in ws], [gpu(b) if b is not None else None for b in bs])
    ref = torch.cat([O.linear(f32(x), f32(w), f32(b) if b is not None else None) for w, b in zip(ws, bs)], dim=-1)
    assert_bf16_close(y, ref, what=f"matmul_segments M={M} {ns}")
    # each column slice equals the single-weight GEMM bit for bit (same kernel math)
    col = 0
    for w, b in zip(ws, bs):
        single = K.matmul(gpu(x), gpu(w), gpu(b) if b is not None else None)
        assert torch.equal(y[:, col:col + w.shape[0]].cpu(), single.cpu()), f"segment at column {col}"
        col += w.shape[0]


@pytest.mark.parametrize("M", [1, 17, 32])
def test_decode_gemv_shapes(M):
    """The C3 decode projections (M <= 32 rows): q/k/v as three segments, o and
    down with the residual fused, gate/up with SwiGLU, at the layer's N and K."""
    H, I = 4096, 12288
    x, xi = rnd(M, H, seed=70), rnd(M, I, seed=71)
    wq, wk, wv = rnd(4096, H, seed=72, std=0.02), rnd(1024, H, seed=73, std=0.02), rnd(1024, H, seed=74, std=0.02)
    y = K.matmul_segments(gpu(x), [gpu(wq), gpu(wk), gpu(wv)])
    ref = torch.cat([O.linear(f32(x), f32(w)) for w in (wq, wk, wv)], dim=-1)
    assert_bf16_close(y, ref, what=f"decode qkv M={M}")
    wo, r = rnd(H, H, seed=75, std=0.02), rnd(M, H, seed=76)
    assert_bf16_close(K.matmul(gpu(x), gpu(wo), residual=gpu(r)), O.linear(f32(x), f32(wo)) + f32(r),
                      what=f"decode o+residual M={M}")
    # gate/up values reach |4..8| here, where half a bf16 ulp of the output
    # alone exceeds 2e-2: bound the worst element by the reference's own bf16
    # path (bf16 gate and up, then swiglu, rounded), as the layer tests do.
    wg, wu = rnd(I, H, seed=77, std=0.02), rnd(I, H, seed=78, std=0.02)
    g32, u32 = O.linear(f32(x), f32(wg)), O.linear(f32(x), f32(wu))
    assert_layer_parity(K.matmul_swiglu(gpu(x), gpu(wg), gpu(wu)), O.swiglu(g32, u32),
                        bf16_round(O.swiglu(bf16_round(g32), bf16_round(u32))), what=f"decode gate/up M={M}")
    wd = rnd(H, I, seed=79, std=0.02)  # K = 12288: outputs reach |10|, same bound as gate/up
    d32 = O.linear(f32(xi), f32(wd))
    assert_layer_parity(K.matmul(gpu(xi), gpu(wd), residual=gpu(r)), d32 + f32(r),
                        bf16_round(bf16_round(d32) + f32(r)), what=f"decode down+residual M={M}")


@pytest.mark.parametrize("M,ns,Kd,kind", [
    (9, (1024, 256, 256), 520, "bias"),    # X staged (one 16-row group), K tail inside a 32-step
    (3, (20000,), 1032, "residual"),       # X direct; 64-row blocks, more blocks than CUs
    (24, (1002,), 4104, "bias"),           # X staged (two groups); N % 4 != 0 (scalar stores)
    (12, (700,), 1000, "swiglu"),          # SwiGLU, X staged, ragged K chunk
    (8, (4096,), 2048, "residual"),        # last M of the direct-X kernel
    (32, (128,), 2048, "plain"),           # router-sized: 8 rows per block, 16 blocks
    (17, (1024,), 16400, "residual"),      # M > 8, K > 16384: the stream-K kernel
    (17, (512,), 16384, "swiglu"),         # last K of the row-owned kernel
    (20, (16000,), 2056, "residual"),      # 63 rows per block (4 row groups, 128-k stages), K tail
    (13, (10000,), 1000, "bias"),          # 40 rows per block (3 row groups), one X tile
    (30, (3000,), 1160, "swiglu"),         # 12 gate + 12 up rows per block, K tail inside a stage
])
def test_gemv_edges(M, ns, Kd, kind):
    """Decode shapes (M <= 32) on the row-owned GEMV (M <= 8, or K <= 16384) and
    the stream-K one: ragged rows, K tails, segments with bias, residual,
    SwiGLU; and run-to-run identity. Weights ~N(0, 1/K) keep the outputs near
    unit scale, where half a bf16 ulp stays inside the 2e-2 bound."""
    sd = Kd ** -0.5
    x = rnd(M, Kd, seed=90)
    if kind == "swiglu":
        wg, wu = rnd(ns[0], Kd, seed=91, std=sd), rnd(ns[0], Kd, seed=92, std=sd)
        y = K.matmul_swiglu(gpu(x), gpu(wg), gpu(wu))
        ref = O.swiglu(O.linear(f32(x), f32(wg)), O.linear(f32(x), f32(wu)))
        again = K.matmul_swiglu(gpu(x), gpu(wg), gpu(wu))
    elif len(ns) > 1:
        ws = [rnd(n, Kd, seed=93 + i, std=sd) for i, n in enumerate(ns)]
        bs = [rnd(n, seed=97 + i, std=sd) for i, n in enumerate(ns)]
        y = K.matmul_segments(gpu(x), [gpu(w) for w in ws], [gpu(b) for b in bs])
        ref = torch.cat([O.linear(f32(x), f32(w), f32(b)) for w, b in zip(ws, bs)], dim=-1)
        again = K.matmul_segments(gpu(x), [gpu(w) for w in ws], [gpu(b) for b in bs])
    else:
        w = rnd(ns[0], Kd, seed=94, std=sd)
        b = rnd(ns[0], seed=95, std=sd) if kind == "bias" else None
        r = rnd(M, ns[0], seed=96) if kind == "residual" else None
        y = K.matmul(gpu(x), gpu(w), gpu(b) if b is not None else None,
                     residual=gpu(r) if r is not None else None)
        ref = O.linear(f32(x), f32(w), f32(b) if b is not None else None) + (f32(r) if r is not None else 0)
        again = K.matmul(gpu(x), gpu(w), gpu(b) if b is not None else None,
                         residual=gpu(r) if r is not None else None)
    assert_bf16_close(y, ref, what=f"gemv M={M} N={ns} K={Kd} {kind}")
    assert torch.equal(y.cpu(), again.cpu()), "the GEMV must be deterministic"


@pytest.mark.parametrize("M,ns,Kd,kind", [
    (32, (4096, 1024, 1024), 4096, "plain"),  # the decode q/k/v shape (B=32)
    (1, (256,), 520, "bias"),                  # one row, K tail inside a chunk
    (9, (1000, 24), 1032, "bias"),             # ragged segments, K tail
    (17, (384,), 2048, "swiglu"),
    (32, (12288,), 4096, "swiglu"),            # the decode gate/up shape (B=32)
    (5, (200,), 4104, "swiglu"),               # M <= 8 also stages X when fused
    (32, (512,), 20480, "plain"),              # K past the row-owned limit: still row-owned
    (32, (6000,), 8192, "plain"),              # the norm weight's LDS copy at its largest K
    (20, (3000,), 8200, "swiglu"),             # K past it: the norm staged through registers
    (12, (16000,), 2056, "bias"),              # 63 rows per block, one X tile, K tail
])
def test_rmsnorm_matmul_fused(M, ns, Kd, kind):
    """RMSNorm fused into the decode projection (q3_rmsnorm_matmul_segments /
    q3_rmsnorm_matmul_swiglu) against the fp32 oracle's rmsnorm -> linear
    (-> swiglu), with the worst element bounded as in the layer tests by the
    reference's own bf16 path (norm output, projections and swiglu each
    rounded to bf16); against the two-launch library path; run-to-run
    identity. Inputs at 3x unit scale make the norm's 1/rms factor matter."""
    eps = 1e-6
    sd = Kd ** -0.5
    x = rnd(M, Kd, seed=100, std=3.0)
    nw = (1.0 + rnd(Kd, seed=101, std=0.2, dtype=torch.float32)).to(torch.bfloat16)
    xn = O.rmsnorm(f32(x), f32(nw), eps)
    xb = bf16_round(xn)
    if kind == "swiglu":
        wg, wu = rnd(ns[0], Kd, seed=102, std=sd), rnd(ns[0], Kd, seed=103, std=sd)
        call = lambda: K.rmsnorm_matmul_swiglu(gpu(x), gpu(nw), eps, gpu(wg), gpu(wu))
        ref = O.swiglu(O.linear(xn, f32(wg)), O.linear(xn, f32(wu)))
        ref_bf16 = bf16_round(O.swiglu(bf16_round(O.linear(xb, f32(wg))), bf16_round(O.linear(xb, f32(wu)))))
        two = K.matmul_swiglu(K.rmsnorm(gpu(x), gpu(nw), eps), gpu(wg), gpu(wu))
    else:
        ws = [rnd(n, Kd, seed=104 + i, std=sd) for i, n in enumerate(ns)]
        bs = [rnd(n, seed=108 + i, std=sd) if kind == "bias" else None for i, n in enumerate(ns)]
        gb = [gpu(b) if b is not None else None for b in bs]
        call = lambda: K.rmsnorm_matmul_segments(gpu(x), gpu(nw), eps, [gpu(w) for w in ws], gb)
        fb = [f32(b) if b is not None else None for b in bs]
        ref = torch.cat([O.linear(xn, f32(w), b) for w, b in zip(ws, fb)], dim=-1)
        ref_bf16 = bf16_round(torch.cat([O.linear(xb, f32(w), b) for w, b in zip(ws, fb)], dim=-1))
        two = K.matmul_segments(K.rmsnorm(gpu(x), gpu(nw), eps), [gpu(w) for w in ws], gb)
    y = call()
    assert y.shape == ref.shape and y.dtype == torch.bfloat16
    assert_layer_parity(y, ref, ref_bf16, what=f"rmsnorm+{kind} M={M} K={Kd}")
    # The two-launch library path meets the same bar against fp32.
    assert_layer_parity(two, ref, ref_bf16, what=f"two launches M={M} K={Kd}")
    assert torch.equal(y, call()), "fused norm projection must be deterministic"


def test_rmsnorm_matmul_fused_closed_forms():
    """Pins that do not go through the oracle: a constant row c*1 with eps = 0
    normalises to sign(c)*w exactly, so the projection equals (sign(c)*w).W^T
    (one bf16 rounding of w*x per element, here exact: x is a power of two);
    K = 8 (one 16-byte piece) and a single row."""
    Kd, N = 1024, 384
    nw = (1.0 + rnd(Kd, seed=120, std=0.2, dtype=torch.float32)).to(torch.bfloat16)
    w = rnd(N, Kd, seed=121, std=Kd ** -0.5)
    x = torch.full((3, Kd), 4.0).to(torch.bfloat16)
    x[1] = -0.5
    x[2] = 2.0 ** -6
    y = K.rmsnorm_matmul_segments(gpu(x), gpu(nw), 0.0, [gpu(w)])
    sign = torch.tensor([1.0, -1.0, 1.0]).unsqueeze(1)
    ref = sign * O.linear(f32(nw).unsqueeze(0), f32(w))
    assert_bf16_close(y, ref, what="constant rows, eps=0")
    # The row scale enters only through rsqrt(mean(x^2)) (hardware reciprocal
    # square root): outputs agree to a bf16 ulp across scales and signs.
    assert_within_ulp(y[2], y[0].float(), ulps=1, what="constant row: scale invariance")
    assert_within_ulp(y[1], -y[0].float(), ulps=1, what="constant row: sign")
    # K = 8: one piece of one chunk, one row
    x8, nw8, w8 = rnd(1, 8, seed=122), rnd(8, seed=123, std=0.1) + 1, rnd(40, 8, seed=124)
    y8 = K.rmsnorm_matmul_segments(gpu(x8), gpu(nw8.to(torch.bfloat16)), 1e-6, [gpu(w8)])
    ref8 = O.linear(O.rmsnorm(f32(x8), f32(nw8.to(torch.bfloat16)), 1e-6), f32(w8))
    assert_bf16_close(y8, ref8, what="K=8")


def test_rmsnorm_matmul_fused_rejects_prefill_rows():
    x = gpu(rnd(33, 64))
    with pytest.raises(ValueError):
        K.rmsnorm_matmul_segments(x, gpu(rnd(64)), 1e-6, [gpu(rnd(16, 64))])


def test_matmul_fp32_reference_style():
    torch.manual_seed(0)
    x, w, b = torch.randn(8, 64), torch.randn(32, 64), torch.randn(32)
    y = K.matmul(gpu(x), gpu(w), gpu(b))
    assert_close(y, O.linear(x, w, b), atol=1e-3, what="fp32 matmul")


def test_matmul_identity():
    x = rnd(64, 256, seed=10)
    eye = torch.eye(256, dtype=torch.bfloat16)
    y = K.matmul(gpu(x), gpu(eye))
    assert torch.equal(y.cpu(), x), "x . I must reproduce x exactly"


@pytest.mark.parametrize("E,M,N,K_", [(4, 8, 12, 16), (8, 96, 256, 512), (3, 40, 72, 64)])
def test_batched_gemm(E, M, N, K_):
    x, w = rnd(E, M, K_, seed=11), rnd(E, N, K_, seed=12, std=0.02)
    y = K.cuda_batched_gemm(gpu(x), gpu(w))
    assert_bf16_close(y, O.batched_gemm(f32(x), f32(w)), what="batched_gemm")
    xf, wf = f32(x), f32(w)
    yf = K.cuda_batched_gemm(gpu(xf), gpu(wf))
    assert_close(yf, O.batched_gemm(xf, wf), atol=1e-3, what="fp32 batched_gemm")


def test_conv3d_patch():
    x = (torch.rand(64, 3, 2, 16, 16, generator=torch.Generator().manual_seed(13)) * 2 - 1).to(torch.bfloat16)
    w, b = rnd(1152, 3, 2, 16, 16, seed=14, std=0.02), rnd(1152, seed=15, std=0.02)
    y = K.conv3d_patch(gpu(x), gpu(w), gpu(b))
    assert_bf16_close(y, O.conv3d_patch(f32(x), f32(w), f32(b)), what="conv3d_patch")
    # the reference's test shape, fp32 (tests/test_kernels.py:313-325)
    xs, ws, bs = torch.randn(4, 3, 2, 16, 16), torch.randn(32, 3, 2, 16, 16), torch.randn(32)
    assert_close(K.conv3d_patch(gpu(xs), gpu(ws), gpu(bs)), O.conv3d_patch(xs, ws, bs), atol=5e-2, what="fp32 conv")


# ------------------------------------------------------------------ attention
@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal", [
    (1, 8, 2, 300, 128, True),
    (2, 4, 1, 130, 128, True),
    (1, 32, 8, 512, 128, True),
    (1, 8, 2, 1100, 128, False),  # odd number of key tiles, ragged last tile
    (1, 4, 1, 1000, 128, True),
    (1, 4, 4, 200, 128, False),  # one head per KV head: 4 query tiles per block
    (1, 4, 2, 100, 128, True),   # groups 2
    (2, 4, 4, 200, 64, False),
    (4, 4, 4, 784, 72, False),   # vision: head_dim 72, per-image
    (1, 2, 2, 77, 80, True),
    (1, 6, 2, 64, 96, False),
    # the eight-wave pipelined kernel's other forms: causal MHA (groups 1, Sq >= 192), whose
    # 256-query blocks have waves with up to 7 fully masked key tiles, and GQA groups 4 at
    # the padded head dims (72, 80, 96)
    (1, 4, 4, 300, 128, True),
    (1, 4, 4, 300, 64, True),
    (2, 3, 3, 520, 128, True),
    (1, 8, 2, 300, 72, True),
    (1, 8, 2, 300, 72, False),
    (1, 8, 2, 260, 80, True),
    (1, 8, 2, 260, 80, False),
    (1, 8, 2, 333, 96, True),
    (1, 8, 2, 333, 96, False),
])
def test_flash_attention_bf16(B, Hq, Hkv, S, D, causal):
    q, k, v = rnd(B, Hq, S, D, seed=20), rnd(B, Hkv, S, D, seed=21), rnd(B, Hkv, S, D, seed=22)
    scale = D ** -0.5
    o = K.flash_attention(gpu(q), gpu(k), gpu(v), scale, causal, Hq // Hkv)
    ref = O.flash_attention(f32(q), f32(k), f32(v), scale, causal, Hq // Hkv)
    assert_bf16_close(o, ref, what=f"flash {B},{Hq},{Hkv},{S},{D},{causal}")


def test_flash_attention_strided_views_and_out():
    B, S, Hq, Hkv, D = 2, 96, 8, 2, 128
    qs, ks, vs = rnd(B, S, Hq, D, seed=23), rnd(B, S, Hkv, D, seed=24), rnd(B, S, Hkv, D, seed=25)
    out = torch.empty(B, S, Hq, D, dtype=torch.bfloat16, device=DEV)
    K.flash_attention(gpu(qs).transpose(1, 2), gpu(ks).transpose(1, 2), gpu(vs).transpose(1, 2), D ** -0.5, True,
                      4, out=out.transpose(1, 2))
    ref = O.flash_attention(f32(qs).transpose(1, 2), f32(ks).transpose(1, 2), f32(vs).transpose(1, 2), D ** -0.5,
                            True, 4)
    assert_bf16_close(out.transpose(1, 2), ref, what="strided flash")


@pytest.mark.parametrize("causal", [True, False])
def test_flash_attention_sharp_scores(causal):
    """Large logits (scale 1 at D=128): the running max keeps rising over key tiles."""
    B, Hq, Hkv, S, D = 1, 8, 2, 640, 128
    q, k, v = rnd(B, Hq, S, D, seed=32), rnd(B, Hkv, S, D, seed=33), rnd(B, Hkv, S, D, seed=34)
    # keys whose norm grows with the index make later tiles dominate
    k = (k.float() * torch.linspace(0.2, 1.5, S).view(1, 1, S, 1)).to(torch.bfloat16)
    # a sharp softmax returns nearly single rows of v: keep |v| < 2 so one bf16
    # output rounding stays well inside the tolerance
    v = (v.float() * 0.5).to(torch.bfloat16)
    o = K.flash_attention(gpu(q), gpu(k), gpu(v), 1.0, causal, Hq // Hkv)
    ref = O.flash_attention(f32(q), f32(k), f32(v), 1.0, causal, Hq // Hkv)
    assert_bf16_close(o, ref, what=f"sharp flash causal={causal}")


def test_flash_attention_causal_row0_is_v0():
    q, k, v = rnd(1, 4, 64, 128, seed=26), rnd(1, 4, 64, 128, seed=27), rnd(1, 4, 64, 128, seed=28)
    o = K.flash_attention(gpu(q), gpu(k), gpu(v), 0.1, True, 1)
    assert torch.equal(o[:, :, 0].cpu(), v[:, :, 0]), "causal row 0 attends only to key 0"


@pytest.mark.parametrize("causal,groups", [(True, 1), (False, 1), (True, 2)])
def test_flash_attention_fp32_reference_style(causal, groups):
    torch.manual_seed(42)
    q = torch.randn(2, 4 * groups, 16, 32)
    k, v = torch.randn(2, 4, 16, 32), torch.randn(2, 4, 16, 32)
    o = K.flash_attention(gpu(q), gpu(k), gpu(v), 32 ** -0.5, causal, groups)
    assert_close(o, O.flash_attention(q, k, v, 32 ** -0.5, causal, groups), atol=1e-3, what="fp32 flash")


def test_flash_attention_sq_ne_sk_noncausal():
    q, k, v = rnd(1, 8, 5, 128, seed=29), rnd(1, 2, 300, 128, seed=30), rnd(1, 2, 300, 128, seed=31)
    o = K.flash_attention(gpu(q), gpu(k), gpu(v), 128 ** -0.5, False, 4)
    assert_bf16_close(o, O.flash_attention(f32(q), f32(k), f32(v), 128 ** -0.5, False, 4), what="Sq != Sk")


@pytest.mark.parametrize("groups", [1, 3, 4, 8, 16])
def test_decode_attention_ragged(groups):
    B, Hkv, cap, D = 7, 2, 1100, 128
    lens = torch.tensor([1, 5, 0, 255, 256, 257, 1100], dtype=torch.int32)
    q = rnd(B, Hkv * groups, D, seed=32)
    kc, vc = rnd(B, Hkv, cap, D, seed=33), rnd(B, Hkv, cap, D, seed=34)
    o = K.decode_attention(gpu(q), gpu(kc), gpu(vc), gpu(lens), D ** -0.5)
    ref = O.decode_attention(f32(q)[:, :, None], f32(kc), f32(vc), lens, D ** -0.5, groups)[:, :, 0]
    assert_bf16_close(o, ref, what=f"decode groups={groups}")


def test_decode_attention_append_step():
    # the new token's row is already at cache row lens[b]: attend to lens + 1 rows, then lens += 1
    B, Hkv, G, D, cap = 5, 2, 4, 128, 300
    lens = torch.tensor([0, 3, 64, 100, 299], dtype=torch.int32)
    q = rnd(B, Hkv * G, D, seed=35)
    kc, vc = rnd(B, Hkv, cap, D, seed=36), rnd(B, Hkv, cap, D, seed=37)
    lens_d = gpu(lens)
    o = K.decode_attention(gpu(q), gpu(kc), gpu(vc), lens_d, D ** -0.5, append=True)
    assert torch.equal(lens_d.cpu(), lens + 1)
    ref = O.decode_attention(f32(q)[:, :, None], f32(kc), f32(vc), lens + 1, D ** -0.5, G)[:, :, 0]
    assert_bf16_close(o, ref, what="decode append step")


def test_decode_attention_c3_lengths():
    # the C3 decode shape: 32 sequences x 8 KV heads, lengths U[1024, 8192] (a work split where
    # pairs straddle waves), plus a second call with most sequences short (pairs inside one wave)
    B, Hkv, G, D, cap = 32, 8, 4, 128, 8193
    g = torch.Generator().manual_seed(0)
    gd = torch.Generator(device="cuda").manual_seed(0)
    kd = torch.randn(B, Hkv, cap, D, generator=gd, device="cuda").to(torch.bfloat16)
    vd = torch.randn(B, Hkv, cap, D, generator=gd, device="cuda").to(torch.bfloat16)
    q = torch.randn(B, Hkv * G, D, generator=g).to(torch.bfloat16)
    qd = gpu(q)
    for lens in (torch.randint(1024, 8193, (B,), generator=g, dtype=torch.int32),
                 torch.randint(1, 40, (B,), generator=g, dtype=torch.int32)):
        o = K.decode_attention(qd, kd, vd, gpu(lens), D ** -0.5).float().cpu()
        for b in (0, 7, 31):  # per-sequence fp32 reference on a sample of sequences
            L = int(lens[b])
            kb, vb = kd[b:b + 1, :, :L].float().cpu(), vd[b:b + 1, :, :L].float().cpu()
            ref = O.flash_attention(q[b:b + 1, :, None].float(), kb, vb, D ** -0.5, False, G)[0, :, 0]
            assert_bf16_close(o[b], ref, what=f"C3 decode b={b} L={L}")


# ------------------------------------------------------------------ rotary
def test_apply_mrope_matches_oracle():
    B, H, S, D = 2, 4, 50, 128
    x = rnd(B, H, S, D, seed=40)
    pos = torch.stack([torch.arange(S), torch.arange(S) * 2, torch.arange(S) * 3]).view(3, 1, S).expand(3, B, S)
    cos3, sin3 = O.mrope_cos_sin(pos, D, 5e6)
    y = K.apply_mrope(gpu(x), gpu(cos3), gpu(sin3), [24, 20, 20])
    assert_bf16_close(y, O.apply_mrope(f32(x), cos3, sin3, [24, 20, 20]), what="apply_mrope")


def test_apply_rope_2d_and_broadcast():
    B, H, S, D = 4, 16, 784, 72
    x = rnd(B, H, S, D, seed=41)
    ang = torch.rand(S, 36, generator=torch.Generator().manual_seed(42)) * 20
    emb = torch.cat([ang, ang], -1)
    cos, sin = emb.cos(), emb.sin()
    ref = O.apply_rope(f32(x), cos, sin)
    assert_bf16_close(K.apply_rope(gpu(x), gpu(cos), gpu(sin)), ref, what="rope 2d cos")
    assert_bf16_close(K.apply_rope(gpu(x), gpu(cos[None]), gpu(sin[None])), ref, what="rope (1,S,D) cos")


def test_apply_rope_partial_dims_fp32():
    torch.manual_seed(0)
    x = torch.randn(2, 3, 10, 32)
    ang = torch.randn(10, 8)
    cos, sin = torch.cat([ang, ang], -1).cos(), torch.cat([ang, ang], -1).sin()
    y = K.apply_rope(gpu(x), gpu(cos), gpu(sin))
    assert_close(y, O.apply_rope(x, cos, sin), atol=1e-5, what="partial rope")


@pytest.mark.parametrize("D,section", [(128, [24, 20, 20]), (64, [12, 10, 10])])
def test_qk_norm_rope_fused(D, section):
    B, S, Hq, Hkv = 2, 40, 8, 2
    q, k, v = rnd(B, S, Hq, D, seed=43), rnd(B, S, Hkv, D, seed=44), rnd(B, S, Hkv, D, seed=45)
    qw, kw = rnd(D, seed=46, std=0.1) + 1, rnd(D, seed=47, std=0.1) + 1
    pos = torch.stack([torch.arange(S) + 3, torch.arange(S) * 2, torch.arange(S) + 7]).view(3, 1, S).expand(3, B, S)
    rope_if = O.mrope_inv_freq(D, 5e6)
    qo, ko, vo = (torch.empty_like(t, device=DEV) for t in (q, k, v))
    K.qk_norm_rope(gpu(q), gpu(k), gpu(v), qo, ko, vo, gpu(qw), gpu(kw), gpu(pos.to(torch.int32).contiguous()),
                   gpu(rope_if), section, 1e-6)
    cos3, sin3 = O.mrope_cos_sin(pos, D, 5e6)
    qr = O.apply_mrope(O.rmsnorm(f32(q), f32(qw)).transpose(1, 2), cos3, sin3, section).transpose(1, 2)
    kr = O.apply_mrope(O.rmsnorm(f32(k), f32(kw)).transpose(1, 2), cos3, sin3, section).transpose(1, 2)
    assert_bf16_close(qo, qr, what="fused q")
    assert_bf16_close(ko, kr, what="fused k")
    assert torch.equal(vo.cpu(), v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_qk_norm_rope_decode_rows_split(dtype):
    """A decode step's q/k/v rows (32 + 8 + 8 heads of 128: three 16-row passes per token) run
    as parallel blocks per token; each block's rows must match the oracle, cache offsets too."""
    B, Hq, Hkv, D, cap = 5, 32, 8, 128, 24
    q, k, v = rnd(B, 1, Hq, D, seed=80, dtype=dtype), rnd(B, 1, Hkv, D, seed=81, dtype=dtype), \
        rnd(B, 1, Hkv, D, seed=82, dtype=dtype)
    qw, kw = (rnd(D, seed=83, std=0.1) + 1).to(dtype), (rnd(D, seed=84, std=0.1) + 1).to(dtype)
    lens = torch.tensor([0, 3, 17, 9, 23], dtype=torch.int32)
    pos = lens.view(1, B, 1).expand(3, B, 1).contiguous()
    qo = torch.empty(B, 1, Hq, D, dtype=dtype, device=DEV)
    kc = torch.zeros(B, cap, Hkv, D, dtype=dtype, device=DEV)
    vc = torch.zeros_like(kc)
    K.qk_norm_rope(gpu(q), gpu(k), gpu(v), qo, kc, vc, gpu(qw), gpu(kw), gpu(pos.to(torch.int32)),
                   gpu(O.mrope_inv_freq(D, 5e6)), (24, 20, 20), 1e-6, dst_seq_offset=gpu(lens), dst_seq_cap=cap)
    cos3, sin3 = O.mrope_cos_sin(pos, D, 5e6)
    qr = O.apply_mrope(O.rmsnorm(f32(q), f32(qw)).transpose(1, 2), cos3, sin3, (24, 20, 20)).transpose(1, 2)
    kr = O.apply_mrope(O.rmsnorm(f32(k), f32(kw)).transpose(1, 2), cos3, sin3, (24, 20, 20)).transpose(1, 2)
    check = assert_bf16_close if dtype == torch.bfloat16 else (lambda o, r, what: assert_close(o, r, 1e-4, what=what))
    check(qo, qr, what="decode q rows")
    kcc, vcc = kc.cpu(), vc.cpu()
    for b in range(B):
        check(kcc[b, int(lens[b])], kr[b, 0], what=f"decode k row of sequence {b}")
        assert torch.equal(vcc[b, int(lens[b])], v[b, 0]), f"v row of sequence {b}"
        others = [r for r in range(cap) if r != int(lens[b])]
        assert not kcc[b, others].any() and not vcc[b, others].any(), "only the appended row is written"


@pytest.mark.parametrize("B,S,Hq,Hkv,D,section,causal", [
    (2, 300, 16, 4, 128, (24, 20, 20), True),   # ragged last query tile
    (1, 256, 32, 4, 128, (24, 20, 20), True),   # groups 8 (C4's)
    (2, 130, 8, 1, 64, (12, 10, 10), False),
    (1, 64, 8, 2, 128, (24, 20, 20), False),  # one query tile, non-causal
    (1, 253, 8, 2, 128, (24, 20, 20), True),  # token count not a multiple of the k kernel's 4 per block
])
def test_qk_norm_rope_attention(B, S, Hq, Hkv, D, section, causal):
    """q/k norm + mRoPE + attention in two launches (q rotated inside the attention kernel) against
    the fp32 oracle chain, and against qk_norm_rope followed by flash_attention on the same views."""
    N = (Hq + 2 * Hkv) * D
    qkv = rnd(B, S, N, seed=60)
    qw, kw = rnd(D, seed=61, std=0.1) + 1, rnd(D, seed=62, std=0.1) + 1
    pos = torch.stack([torch.arange(S) + 5, torch.arange(S) // 3, torch.arange(S) % 17]).view(3, 1, S).expand(3, B, S)
    pos_d = gpu(pos.to(torch.int32).contiguous())
    inv = gpu(O.mrope_inv_freq(D, 5e6))
    scale = D ** -0.5

    def views(t):
        return (t[..., :Hq * D].view(B, S, Hq, D), t[..., Hq * D:(Hq + Hkv) * D].view(B, S, Hkv, D),
                t[..., (Hq + Hkv) * D:].view(B, S, Hkv, D))
    fused_buf = gpu(qkv)
    q, k, v = views(fused_buf)
    o = K.qk_norm_rope_attention(q, k, v, gpu(qw), gpu(kw), pos_d, inv, section, 1e-6, scale, causal)
    assert torch.equal(fused_buf[..., :Hq * D].cpu(), qkv[..., :Hq * D]), "q_in must not be modified"

    two_buf = gpu(qkv)
    q2, k2, v2 = views(two_buf)
    qk_out = torch.empty_like(q2)
    K.qk_norm_rope(q2, k2, None, qk_out, k2, None, gpu(qw), gpu(kw), pos_d, inv, section, 1e-6)
    o2 = K.flash_attention(qk_out.transpose(1, 2), k2.transpose(1, 2), v2.transpose(1, 2), scale, causal,
                           Hq // Hkv).transpose(1, 2)
    assert torch.equal(k.cpu(), k2.cpu()), "k rows: the same kernel code as qk_norm_rope"
    # q may differ from the separate kernel's by one bf16 ulp in rare elements (sum-of-squares order)
    assert (o.float() - o2.float()).abs().max().item() <= 4e-3

    cos3, sin3 = O.mrope_cos_sin(pos, D, 5e6)
    qs, ks, vs = views(f32(qkv))
    qr = O.apply_mrope(O.rmsnorm(qs, f32(qw)).transpose(1, 2), cos3, sin3, section)
    kr = O.apply_mrope(O.rmsnorm(ks, f32(kw)).transpose(1, 2), cos3, sin3, section)
    ref = O.flash_attention(qr, kr, vs.transpose(1, 2), scale, causal, Hq // Hkv).transpose(1, 2)
    assert_bf16_close(k, kr.transpose(1, 2), what="fused k rows")
    assert_bf16_close(o, ref, what=f"qk_norm_rope_attention {B},{S},{Hq},{Hkv},{D}")


# ------------------------------------------------------------------ norms / elementwise
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (2048, 128), (100, 1152), (33, 2048), (17, 37), (8, 256)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rmsnorm(rows, cols, dtype):
    x, w = rnd(rows, cols, seed=50, dtype=dtype), rnd(cols, seed=51, std=0.2, dtype=dtype) + 1
    y = K.rmsnorm(gpu(x), gpu(w), 1e-6)
    ref = O.rmsnorm(f32(x), f32(w), 1e-6)
    if dtype == torch.float32:
        assert_close(y, ref, atol=1e-4, what="fp32 rmsnorm")
    else:
        assert_bf16_close(y, ref, what="rmsnorm")


def test_rmsnorm_constant_row_equals_weight():
    x = torch.full((4, 4096), 3.0, dtype=torch.bfloat16)
    w = rnd(4096, seed=52, std=0.5)
    y = K.rmsnorm(gpu(x), gpu(w), 0.0)
    assert_bf16_close(y, f32(w).expand(4, -1), max_abs=1e-2, what="rms(const) == w")


@pytest.mark.parametrize("rows,cols", [(3136, 1152), (64, 64), (10, 100)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_layernorm(rows, cols, dtype):
    x = rnd(rows, cols, seed=53, dtype=dtype) * 3 + 2
    w, b = rnd(cols, seed=54, std=0.2, dtype=dtype) + 1, rnd(cols, seed=55, std=0.2, dtype=dtype)
    y = K.layernorm(gpu(x), gpu(w), gpu(b), 1e-6)
    ref = O.layernorm(f32(x), f32(w), f32(b), 1e-6)
    if dtype == torch.float32:
        assert_close(y, ref, atol=1e-4, what="fp32 layernorm")
    else:
        assert_bf16_close(y, ref, what="layernorm")


@pytest.mark.parametrize("n", [1, 7, 4096 * 12288 // 16, 1000003])
def test_elementwise(n):
    # one fp32 computation and one rounding per element: within 1 bf16 ulp of the fp32 oracle
    a, b = rnd(n, seed=56), rnd(n, seed=57)
    assert_within_ulp(K.residual_add(gpu(a), gpu(b)), f32(a) + f32(b), what="residual_add")
    assert_within_ulp(K.swiglu(gpu(a), gpu(b)), O.swiglu(f32(a), f32(b)), what="swiglu")
    assert_within_ulp(K.gelu_tanh(gpu(a)), O.gelu_tanh(f32(a)), what="gelu_tanh")


def test_elementwise_fp32_reference_style():
    torch.manual_seed(0)
    a, b = torch.randn(4, 33), torch.randn(4, 33)
    assert_close(K.residual_add(gpu(a), gpu(b)), a + b, atol=1e-5)
    assert_close(K.swiglu(gpu(a), gpu(b)), O.swiglu(a, b), atol=1e-4)
    assert_close(K.gelu_tanh(gpu(a)), O.gelu_tanh(a), atol=1e-4)


@pytest.mark.parametrize("rows,cols", [(4096, 128), (3, 1000)])
def test_softmax(rows, cols):
    x = torch.randn(rows, cols, generator=torch.Generator().manual_seed(58)) * 3
    assert_close(K.softmax(gpu(x)), O.softmax(x), atol=1e-6, what="softmax")


# ------------------------------------------------------------------ routing
def test_topk_exact_with_planted_ties():
    g = torch.Generator().manual_seed(60)
    x = torch.randint(0, 6, (512, 128), generator=g).float()  # many exact ties
    for k in (1, 4, 8):
        v, i = K.cuda_topk(gpu(x), k)
        rv, ri = O.topk(x, k)
        assert torch.equal(i.cpu(), ri), f"top-{k} indices differ"
        assert torch.equal(v.cpu(), rv)
    # the reference test shape (tests/test_kernels.py:279-285)
    x2 = torch.randn(8, 60, generator=g)
    v, i = K.cuda_topk(gpu(x2), 4)
    rv, ri = O.topk(x2, 4)
    assert torch.equal(i.cpu(), ri) and torch.equal(v.cpu(), rv)


def test_index_add_duplicates_and_order():
    g = torch.Generator().manual_seed(61)
    target = torch.randn(50, 96, generator=g).to(torch.bfloat16)
    src = torch.randn(300, 96, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, 50, (300,), generator=g)
    out = K.cuda_index_add(gpu(target.clone()), gpu(src), gpu(idx))
    ref = O.index_add(target.clone(), src, idx)  # CPU bf16 sequential index_add_
    assert torch.equal(out.cpu(), ref), "bf16 index_add must match the sequential CPU order bit-exactly"
    tf, sf = target.float(), src.float()
    outf = K.cuda_index_add(gpu(tf.clone()), gpu(sf), gpu(idx))
    assert_close(outf, O.index_add(tf.clone(), sf, idx), atol=1e-5, what="fp32 index_add")


def test_moe_route_exact_indices():
    g = torch.Generator().manual_seed(62)
    logits = (torch.randn(4096, 128, generator=g) * 2).to(torch.bfloat16)
    logits[::7, 5] = logits[::7, 9]  # planted exact ties
    idx, w = K.moe_route(gpu(logits), 8, True)
    probs = O.softmax(logits.float())
    rv, ri = O.topk(probs, 8)
    assert torch.equal(idx.cpu().long(), ri), "router top-k indices must be bit-exact"
    assert_bf16_close(w, rv / rv.sum(-1, keepdim=True), max_abs=4e-3, what="routing weights")


@pytest.mark.parametrize("E,k,norm", [(8, 1, True), (8, 8, True), (64, 4, False), (100, 8, True), (256, 32, True),
                                      (500, 16, False), (500, 32, True)])
def test_moe_route_ties_and_widths(E, k, norm):
    """Routing at expert counts of 1-8 registers per lane and k up to 32. The logits are
    multiples of 1/4, so equal logits give exactly equal probabilities (ties, which the
    lower expert index wins) and unequal ones differ by a factor >= e^0.25, which no
    summation order can reorder: the indices are bit-exact against the oracle's top-k."""
    g = torch.Generator().manual_seed(1000 + E + k)
    logits = ((torch.randn(333, E, generator=g) * 2 * 4).round() / 4).to(torch.bfloat16)
    idx, w = K.moe_route(gpu(logits), k, norm)
    probs = O.softmax(logits.float())
    rv, ri = O.topk(probs, k)
    assert torch.equal(idx.cpu().long(), ri), f"top-k indices E={E} k={k}"
    ref = rv / rv.sum(-1, keepdim=True) if norm else rv
    assert_bf16_close(w, ref, max_abs=4e-3, what=f"routing weights E={E} k={k}")


@pytest.mark.parametrize("T,H,E,k", [(4096, 2048, 128, 8), (1000, 2048, 128, 8), (333, 1024, 64, 4), (77, 520, 96, 2)])
def test_moe_router_split_k(T, H, E, k):
    """The router with its logits GEMM split over K: logits against the fp32 oracle's linear,
    within a bf16 ulp of the unsplit GEMM; top-k indices bit-exact against the oracle's softmax +
    top-k on the returned logits; weights as moe_route gives them on the same logits. The last
    shape has H with no 64-column split (one split)."""
    x = rnd(T, H, seed=63, std=1.0)
    wg = rnd(E, H, seed=64, std=H ** -0.5)
    logits, idx, w = K.moe_router(gpu(x), gpu(wg), k, True)
    ref = O.linear(f32(x), f32(wg))
    assert_bf16_close(logits, ref, what=f"router logits T={T} H={H} E={E}")
    # one bf16 ulp of the unsplit result, with an absolute floor for logits near zero, where the
    # two fp32 summation orders differ by more than an ulp of the tiny result (cancellation)
    plain = K.matmul(gpu(x), gpu(wg)).float().cpu()
    ulp = torch.exp2(torch.floor(torch.log2(plain.abs().clamp_min(1e-30))) - 7).clamp_min(2.0 ** -14)
    assert bool(((logits.float().cpu() - plain).abs() <= ulp).all()), "split-K logits within 1 bf16 ulp"
    probs = O.softmax(logits.float().cpu())
    rv, ri = O.topk(probs, k)
    assert torch.equal(idx.cpu().long(), ri), "router top-k indices must be bit-exact"
    idx2, w2 = K.moe_route(logits, k, True)
    assert torch.equal(idx2, idx) and torch.equal(w2, w)


def test_moe_experts_against_oracle_loop():
    from oracle.layers import sparse_moe
    T, H, I, E, k = 256, 256, 128, 16, 4
    g = torch.Generator().manual_seed(63)
    x = torch.randn(1, T, H, generator=g).to(torch.bfloat16)
    p = {"gate_weight": (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16),
         "gate_up_proj": (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16),
         "down_proj": (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)}
    logits = K.matmul(gpu(x[0]), gpu(p["gate_weight"]))
    idx, w = K.moe_route(logits, k, True)
    out = K.moe_experts(gpu(x[0]), gpu(p["gate_up_proj"]), gpu(p["down_proj"]), idx, w)
    pf = {n: f32(t) for n, t in p.items()}
    ref, _ = sparse_moe(f32(x), pf, top_k=k, router_logits=logits.float().cpu())
    assert_bf16_close(out, ref[0], what="moe_experts")


def test_moe_experts_skewed_routing():
    """One expert takes every token (600 rows: m-tiles of 256, 256 and 88 rows, the last with
    an empty upper half), the second choice spreads over the others (~86 rows each)."""
    from oracle.layers import sparse_moe
    T, H, I, E, k = 600, 256, 128, 8, 2
    g = torch.Generator().manual_seed(71)
    x = torch.randn(1, T, H, generator=g).to(torch.bfloat16)
    p = {"gate_weight": (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16),
         "gate_up_proj": (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16),
         "down_proj": (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)}
    logits = torch.randn(T, E, generator=g)
    logits[:, 0] += 10.0
    logits = logits.to(torch.bfloat16)
    idx, w = K.moe_route(gpu(logits), k, True)
    counts = torch.bincount(idx.long().flatten().cpu(), minlength=E)
    assert counts[0].item() == T and counts[1:].sum().item() == T
    out = K.moe_experts(gpu(x[0]), gpu(p["gate_up_proj"]), gpu(p["down_proj"]), idx, w)
    pf = {n: f32(t) for n, t in p.items()}
    ref, _ = sparse_moe(f32(x), pf, top_k=k, router_logits=logits.float())
    assert_bf16_close(out, ref[0], what="moe_experts skewed")



def test_moe_experts_tile_row_counts():
    """Expert row counts on both sides of every 32-row block and 128-row half of a 256-row
    m-tile (a wave of the grouped tiles holds 128 rows as four 32-row blocks, and skips the
    MFMAs of the blocks past its rows), plus one expert that takes every token's second
    choice (2052 rows: eight full m-tiles and one of 4 rows)."""
    from oracle.layers import sparse_moe
    counts = [1, 31, 32, 33, 97, 128, 129, 161, 255, 256, 257, 289, 383]
    E, T, H, I, k = len(counts) + 1, sum(counts), 256, 128, 2
    g = torch.Generator().manual_seed(83)
    x = torch.randn(1, T, H, generator=g).to(torch.bfloat16)
    p = {"gate_weight": (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16),
         "gate_up_proj": (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16),
         "down_proj": (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)}
    first = torch.repeat_interleave(torch.arange(len(counts)), torch.tensor(counts))
    first = first[torch.randperm(T, generator=g)]
    logits = torch.randn(T, E, generator=g)
    logits[torch.arange(T), first] += 18.0
    logits[:, E - 1] += 16.0  # every token's second choice (weights ~0.88 / ~0.12)
    logits = logits.to(torch.bfloat16)
    idx, w = K.moe_route(gpu(logits), k, True)
    assert torch.bincount(idx.long().flatten().cpu(), minlength=E).tolist() == counts + [T]
    out = K.moe_experts(gpu(x[0]), gpu(p["gate_up_proj"]), gpu(p["down_proj"]), idx, w)
    pf = {n: f32(t) for n, t in p.items()}
    ref, _ = sparse_moe(f32(x), pf, top_k=k, router_logits=logits.float())
    assert_bf16_close(out, ref[0], what="moe_experts tile row counts")

# ------------------------------------------------------------------ prefill chunk over a KV cache
@pytest.mark.parametrize("Hq,Hkv,D,dtype,Sq,cap", [
    (8, 2, 128, torch.bfloat16, 77, 300),   # groups 4: the eight-wave pipelined kernel
    (8, 4, 64, torch.bfloat16, 77, 300),    # groups 2: the four-wave kernel family
    (4, 2, 72, torch.bfloat16, 77, 300),    # vision head dim through the same kernel family
    (4, 2, 32, torch.float32, 77, 300),     # fp32: the SIMT kernel
    (4, 4, 128, torch.bfloat16, 200, 520),  # groups 1 with Sq >= 192: the pipelined kernel's MHA form
    (4, 4, 64, torch.bfloat16, 250, 520),
])
def test_flash_attention_cache_ragged(Hq, Hkv, D, dtype, Sq, cap):
    """Chunk of Sq tokens per sequence over cache rows [0, lens[b] + i] (causal over the
    whole sequence), ragged lens incl. 0 and lens + Sq == cap; advance adds Sq in place."""
    B = 4
    lens = torch.tensor([0, 5, min(150, cap - Sq - 1), cap - Sq], dtype=torch.int32)
    q = rnd(B, Hq, Sq, D, seed=200, dtype=dtype)
    kc = rnd(B, Hkv, cap, D, seed=201, dtype=dtype)
    vc = rnd(B, Hkv, cap, D, seed=202, dtype=dtype)
    dl = gpu(lens)
    out = K.flash_attention_cache(gpu(q), gpu(kc), gpu(vc), dl, D ** -0.5, Hq // Hkv, advance=True)
    assert torch.equal(dl.cpu(), lens + Sq), "advance must add Sq to every length"
    ref = O.chunk_attention(f32(q), f32(kc), f32(vc), lens.tolist(), D ** -0.5, Hq // Hkv)
    if dtype == torch.float32:
        assert_close(out, ref, atol=2e-5, what="chunk attention fp32")
    else:
        assert_bf16_close(out, ref, what=f"chunk attention D={D} groups={Hq // Hkv}")
    # Empty cache: plain causal attention over the chunk's own rows, bit for bit where both calls run
    # the same kernel (GQA groups of 4k, fp32); for other groups the cache path runs the pipelined
    # kernel per query head (the kernel of its paged form) and plain attention the four-wave one.
    z = torch.zeros(B, dtype=torch.int32, device=DEV)
    a = K.flash_attention_cache(gpu(q), gpu(kc), gpu(vc), z, D ** -0.5, Hq // Hkv)
    b = K.flash_attention(gpu(q), gpu(kc)[:, :, :Sq], gpu(vc)[:, :, :Sq], D ** -0.5, True, Hq // Hkv)
    if dtype == torch.float32 or (Hq // Hkv) % 4 == 0:
        assert torch.equal(a, b), "an empty cache must give causal attention bit for bit"
    else:
        ref0 = O.flash_attention(f32(q), f32(kc)[:, :, :Sq], f32(vc)[:, :, :Sq], D ** -0.5, True, Hq // Hkv)
        assert_bf16_close(a, ref0, what=f"empty cache, groups {Hq // Hkv}")
    assert torch.equal(z.cpu(), torch.zeros(B, dtype=torch.int32)), "advance=False leaves the lengths"


# ------------------------------------------------------------------ MoE dispatch tables
@pytest.mark.parametrize("T,E,k", [(4096, 128, 8), (300, 16, 4), (70, 64, 1)])
def test_moe_permute_matches_nonzero_order(T, E, k):
    """The dispatch tables against the reference loop's per-expert `(top_idx == e).nonzero()`
    (modules/moe.py:70-76), bit-exact: offsets, the (token) order, routing weights, inverse."""
    g = torch.Generator().manual_seed(210 + T)
    # random distinct experts per token, skewed so some experts get nothing
    scores = torch.rand(T, E, generator=g) * torch.linspace(1.0, 0.05, E)
    top_idx = scores.topk(k, dim=-1).indices.to(torch.int32)
    top_w = torch.rand(T, k, generator=g).to(torch.bfloat16)
    offsets, st, sw, pos_of = K.moe_permute(gpu(top_idx), gpu(top_w), E)
    offsets, st, sw, pos_of = offsets.cpu(), st.cpu(), sw.cpu(), pos_of.cpu()
    row = 0
    for e in range(E):
        tok, slot = (top_idx.long() == e).nonzero(as_tuple=True)
        assert int(offsets[e]) == row, f"offset of expert {e}"
        n = tok.numel()
        assert torch.equal(st[row:row + n].long(), tok), f"token order of expert {e}"
        assert torch.equal(sw[row:row + n], top_w[tok, slot]), f"routing weights of expert {e}"
        assert torch.equal(pos_of[tok, slot].long(), torch.arange(row, row + n)), f"inverse of expert {e}"
        row += n
    assert int(offsets[E]) == row == T * k


def test_index_add_out_of_range_is_skipped_and_flagged():
    """Indices outside [0, rows) are skipped on the device and reported through the status
    word (no host synchronisation in the op); valid rows match the CPU index_add_."""
    from qwen3_5_vl_cuda_custom_amd import _lib
    _lib.device_status(DEV)  # clear anything earlier tests left
    g = torch.Generator().manual_seed(64)
    target = torch.randn(20, 64, generator=g).to(torch.bfloat16)
    src = torch.randn(40, 64, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, 20, (40,), generator=g)
    K.cuda_index_add(gpu(target.clone()), gpu(src), gpu(idx))
    K.raise_device_errors(DEV)  # all in range: nothing recorded
    bad = idx.clone()
    bad[3], bad[17] = 20, -1
    out = K.cuda_index_add(gpu(target.clone()), gpu(src), gpu(bad))
    keep = (bad >= 0) & (bad < 20)
    ref = O.index_add(target.clone(), src[keep], bad[keep])
    assert torch.equal(out.cpu(), ref), "valid rows must be added exactly as before"
    with pytest.raises(IndexError):
        K.raise_device_errors(DEV)
    K.raise_device_errors(DEV)  # the check clears the word


# ------------------------------------------------------------------ slow paths are reported, not silent
def test_unaligned_bf16_operands_run_on_aligned_copies(monkeypatch):
    from qwen3_5_vl_cuda_custom_amd.kernels import _loader
    monkeypatch.delenv("CUDA_QWEN3_VL_STRICT", raising=False)
    _loader.FALLBACK_LOG.clear()
    x, w = rnd(300, 520, seed=300), rnd(264, 520, seed=301)
    xb = torch.empty(300 * 520 + 1, dtype=torch.bfloat16, device=DEV)
    xu = xb[1:].view(300, 520)  # base 2 bytes past the allocation: not 16-byte aligned
    xu.copy_(gpu(x))
    y_al = K.matmul(gpu(x), gpu(w))
    y_un = K.matmul(xu, gpu(w))
    assert torch.equal(y_al, y_un), "the aligned copy must give the aligned call's result"
    assert ("matmul", "aligned_copy", "") in _loader.FALLBACK_LOG
    # attention: a q view at an odd offset
    q, k, v = rnd(1, 8, 96, 128, seed=302), rnd(1, 2, 96, 128, seed=303), rnd(1, 2, 96, 128, seed=304)
    qb = torch.empty(q.numel() + 1, dtype=torch.bfloat16, device=DEV)
    qu = qb[1:].view(q.shape)
    qu.copy_(gpu(q))
    assert torch.equal(K.flash_attention(qu, gpu(k), gpu(v), 0.1, True, 4),
                       K.flash_attention(gpu(q), gpu(k), gpu(v), 0.1, True, 4))
    assert ("flash_attention", "aligned_copy", "") in _loader.FALLBACK_LOG
    # K = 12 (not a multiple of 8): only the SIMT kernel takes it, and that is recorded
    _loader.FALLBACK_LOG.clear()
    a, b = rnd(40, 12, seed=305, std=0.5), rnd(24, 12, seed=306, std=0.5)
    assert_bf16_close(K.matmul(gpu(a), gpu(b)), O.linear(f32(a), f32(b)), what="K=12 SIMT GEMM")
    assert any(op == "matmul" and r.startswith("simt_kernel") for op, r, _ in _loader.FALLBACK_LOG)
    monkeypatch.setenv("CUDA_QWEN3_VL_STRICT", "1")
    with pytest.raises(RuntimeError, match="strict"):
        K.matmul(xu, gpu(w))
    with pytest.raises(RuntimeError, match="strict"):
        K.matmul(gpu(a), gpu(b))
    _loader.FALLBACK_LOG.clear()
