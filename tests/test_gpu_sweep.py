"""Seeded random shapes through the GEMM forms, prefill attention and decode attention,
against the CPU oracle at the literal bar (bf16 max-abs 2e-2, mean-rel 5e-3).

The fixed-shape tests pin the configurations the layers use; these cases reach the
shapes between them: ragged M, N and K (multiples of 8), every epilogue (bias,
residual, SwiGLU, GELU, up to four weight segments), the GEMV rows (M <= 32), head dims
64-128 with GQA groups 1-8, causal and not, and ragged decode caches including empty
sequences. Inputs are scaled so that outputs stay O(1), where one bf16 rounding stays
within the bar. The case list is fixed by its seed, so a failure names a reproducible
case.
"""
import random

import pytest
import torch

from oracle import ops as O
from qwen3_5_vl_cuda_custom_amd import kernels as K
from tests.parity import assert_bf16_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gemm_cases(n, seed):
    r = random.Random(seed)
    out = []
    for _ in range(n):
        M = r.choice([r.randint(1, 32), r.randint(33, 600), r.randint(600, 2100)])
        N = 8 * r.randint(1, 300)
        Kd = 8 * r.randint(1, 300)
        kind = r.choice(["plain", "bias", "res", "bias_res", "swiglu", "gelu", "seg"])
        ns = tuple(8 * r.randint(1, 120) for _ in range(r.randint(2, 4))) if kind == "seg" else ()
        out.append((M, N, Kd, kind, ns, r.randrange(1 << 20)))
    return out


def _attn_cases(n, seed):
    r = random.Random(seed)
    out = []
    for _ in range(n):
        D = r.choice([64, 72, 80, 96, 128])
        Hkv = r.choice([1, 2, 4])
        G = r.choice([1, 2, 4, 8])
        out.append((r.randint(1, 2), Hkv * G, Hkv, r.randint(1, 1200), D, r.random() < 0.6, r.randrange(1 << 20)))
    return out


def _decode_cases(n, seed):
    r = random.Random(seed)
    out = []
    for _ in range(n):
        Hkv = r.choice([1, 2, 4, 8])
        G = r.choice([1, 2, 4, 8, 16, 32])
        out.append((r.randint(1, 40), Hkv * G, Hkv, r.randint(40, 2000), r.randrange(1 << 20)))
    return out


def _rnd(g, *shape, std=1.0):
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


@pytest.mark.parametrize("M,N,Kd,kind,ns,seed", _gemm_cases(24, 2024))
def test_gemm_random_shapes(M, N, Kd, kind, ns, seed):
    g = torch.Generator().manual_seed(seed)
    std = Kd ** -0.5
    x = _rnd(g, M, Kd)
    what = f"{kind} M={M} N={N} K={Kd} {ns}"
    if kind == "swiglu":
        wg, wu = _rnd(g, N, Kd, std=std / 2), _rnd(g, N, Kd, std=std / 2)
        y = K.matmul_swiglu(x.to(DEV), wg.to(DEV), wu.to(DEV))
        ref = O.swiglu(O.linear(x.float(), wg.float()), O.linear(x.float(), wu.float()))
    elif kind == "gelu":
        w, b = _rnd(g, N, Kd, std=std), _rnd(g, N, std=0.02)
        y = K.matmul_gelu(x.to(DEV), w.to(DEV), b.to(DEV))
        ref = O.gelu_tanh(O.linear(x.float(), w.float(), b.float()))
    elif kind == "seg":
        ws = [_rnd(g, n, Kd, std=std) for n in ns]
        bs = [_rnd(g, n, std=0.02) if i % 2 == 0 else None for i, n in enumerate(ns)]
        y = K.matmul_segments(x.to(DEV), [w.to(DEV) for w in ws], [b.to(DEV) if b is not None else None for b in bs])
        ref = torch.cat([O.linear(x.float(), w.float(), b.float() if b is not None else None)
                         for w, b in zip(ws, bs)], dim=-1)
    else:
        w = _rnd(g, N, Kd, std=std)
        b = _rnd(g, N, std=0.02) if "bias" in kind else None
        r = _rnd(g, M, N, std=0.5) if "res" in kind else None
        y = K.matmul(x.to(DEV), w.to(DEV), b.to(DEV) if b is not None else None,
                     residual=r.to(DEV) if r is not None else None)
        ref = O.linear(x.float(), w.float(), b.float() if b is not None else None)
        if r is not None:
            ref = ref + r.float()
    assert_bf16_close(y, ref, what=what)


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal,seed", _attn_cases(10, 2025))
def test_flash_attention_random_shapes(B, Hq, Hkv, S, D, causal, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = _rnd(g, B, Hq, S, D), _rnd(g, B, Hkv, S, D), _rnd(g, B, Hkv, S, D)
    o = K.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), D ** -0.5, causal, Hq // Hkv)
    ref = O.flash_attention(q.float(), k.float(), v.float(), D ** -0.5, causal, Hq // Hkv)
    assert_bf16_close(o, ref, what=f"attention B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal}")


@pytest.mark.parametrize("B,Hq,Hkv,cap,seed", _decode_cases(6, 2026))
def test_decode_attention_random_shapes(B, Hq, Hkv, cap, seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(0, cap + 1, (B,), generator=g, dtype=torch.int32)
    lens[0] = 0  # an empty sequence in every case: its output is zeros
    q, kc, vc = _rnd(g, B, Hq, 128), _rnd(g, B, Hkv, cap, 128), _rnd(g, B, Hkv, cap, 128)
    o = K.decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV), 128 ** -0.5)
    live = (lens > 0).nonzero().flatten()
    ref = torch.zeros(B, Hq, 128)  # an empty cache attends to nothing: zeros (the kernel's contract)
    ref[live] = O.decode_attention(q[live].float().unsqueeze(2), kc[live].float(), vc[live].float(), lens[live],
                                   128 ** -0.5, Hq // Hkv)[:, :, 0]
    assert_bf16_close(o, ref, what=f"decode B={B} Hq={Hq} Hkv={Hkv} cap={cap}")
