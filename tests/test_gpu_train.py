"""The rest of the op namespace (sigmoid_mul, cross_entropy) and the backward of every
differentiable op, through the C-ABI, against torch.autograd on the CPU oracle in fp32.

fp32 cases use the reference's own test shapes and tolerances (tests/test_kernels.py:29-39,
69-79, 109-126, 166-179, 210-250). bf16 cases run at layer sizes; their gradients are
checked relative to the gradient's scale (bf16 rounds every output once: max error within
1.5% of the largest |reference|, mean error within 0.5% of the mean |reference|). Every
backward is also run twice and compared bit for bit (fixed-order reductions, no atomics).
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import ops as O
from qwen3_5_vl_cuda_custom_amd import kernels as K
from tests.parity import assert_bf16_close, assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rnd(*shape, seed=0, std=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def run_grads(fn, inputs, dy, device=DEV, dtype=None):
    """Gradients of sum(fn(*inputs) * dy) w.r.t. the float inputs (computed on `device`)."""
    with torch.enable_grad():
        # fresh leaves every call: .to() alone returns the caller's tensor when nothing changes
        xs = [t.detach().to(device=device, dtype=dtype or t.dtype).clone().requires_grad_(True)
              if t.is_floating_point() else t.to(device) for t in inputs]
        out = fn(*xs)
        out.backward(dy.to(device).to(out.dtype))
    return out.detach(), [x.grad for x in xs if x.is_floating_point()]


def ref_grads(fn, inputs, dy):
    return run_grads(fn, [t.float() if t.is_floating_point() else t for t in inputs], dy.float(), device="cpu")


def assert_grad_close(got, ref, what, max_rel=1.5e-2, mean_rel=5e-3):
    g, r = got.float().cpu(), ref.float().cpu()
    err = (g - r).abs()
    scale = float(r.abs().max())
    assert float(err.max()) <= max_rel * scale + 1e-12, f"{what}: max err {float(err.max()):.3e} vs scale {scale:.3e}"
    assert float(err.mean()) <= mean_rel * float(r.abs().mean()) + 1e-12, f"{what}: mean err {float(err.mean()):.3e}"


def twice_equal(fn):
    a, b = fn(), fn()
    for x, y in zip(a, b):
        assert torch.equal(x, y), "backward must be bitwise reproducible"


# ------------------------------------------------------------------ sigmoid_mul
def test_sigmoid_mul_reference_shapes_fp32():
    x, g = rnd(8, 128, seed=1), rnd(8, 128, seed=2)
    assert_close(K.sigmoid_mul(x.to(DEV), g.to(DEV)), O.sigmoid_mul(x, g), atol=1e-4, what="sigmoid_mul")
    x, g, dy = rnd(4, 64, seed=3), rnd(4, 64, seed=4), rnd(4, 64, seed=5)
    _, (gx, gg) = run_grads(K.sigmoid_mul, [x, g], dy)
    _, (rx, rg) = ref_grads(O.sigmoid_mul, [x, g], dy)
    assert_close(gx, rx, atol=1e-4, what="sigmoid_mul dx")
    assert_close(gg, rg, atol=1e-4, what="sigmoid_mul dgate")


def test_sigmoid_mul_bf16():
    x, g, dy = rnd(64, 1000, seed=6), rnd(64, 1000, seed=7, std=3.0), rnd(64, 1000, seed=8)
    xb, gb = x.bfloat16(), g.bfloat16()
    assert_bf16_close(K.sigmoid_mul(xb.to(DEV), gb.to(DEV)), O.sigmoid_mul(xb.float(), gb.float()), what="sm bf16")
    _, (gx, gg) = run_grads(K.sigmoid_mul, [xb, gb], dy.bfloat16())
    _, (rx, rg) = ref_grads(O.sigmoid_mul, [xb, gb], dy.bfloat16())
    assert_grad_close(gx, rx, "sigmoid_mul dx bf16")
    assert_grad_close(gg, rg, "sigmoid_mul dgate bf16")


# ------------------------------------------------------------------ cross_entropy
@pytest.mark.parametrize("ignore", [False, True])
def test_cross_entropy_reference_shapes_fp32(ignore):
    logits = rnd(16, 100, seed=10)
    tg = torch.randint(0, 100, (16,), generator=torch.Generator().manual_seed(11))
    if ignore:
        tg[[1, 5, 9]] = -100
    loss = K.cross_entropy(logits.to(DEV), tg.to(DEV))
    assert loss.dtype == torch.float32 and loss.dim() == 0
    assert_close(loss, O.cross_entropy(logits, tg), atol=1e-4, what="cross_entropy")
    assert_close(loss, F.cross_entropy(logits, tg), atol=1e-4, what="vs F.cross_entropy")
    with torch.enable_grad():
        lg = logits.to(DEV).requires_grad_(True)
        K.cross_entropy(lg, tg.to(DEV)).backward()
        lr = logits.clone().requires_grad_(True)
        O.cross_entropy(lr, tg).backward()
    assert_close(lg.grad, lr.grad, atol=1e-4, what="cross_entropy grad")


def test_cross_entropy_all_ignored_is_zero_and_grad_scale():
    logits = rnd(8, 50, seed=12).to(DEV)
    tg = torch.full((8,), -100, dtype=torch.int64, device=DEV)
    assert float(K.cross_entropy(logits, tg)) == 0.0
    # an upstream gradient of 3 scales the logits' gradient by 3 (read on the device)
    tg = torch.arange(8, device=DEV)
    with torch.enable_grad():
        a = logits.clone().requires_grad_(True)
        (3.0 * K.cross_entropy(a, tg)).backward()
        b = logits.clone().requires_grad_(True)
        K.cross_entropy(b, tg).backward()
    assert torch.allclose(a.grad, 3.0 * b.grad, rtol=1e-6, atol=0)


def test_cross_entropy_vocab_size_bf16():
    """4096 x 151,936 bf16 logits (the Qwen3-VL vocabulary): loss and sampled gradient rows."""
    N, V = 4096, 151936
    gd = torch.Generator(device=DEV).manual_seed(13)
    logits = (torch.randn(N, V, generator=gd, device=DEV) * 2.0).to(torch.bfloat16)
    tg = torch.randint(0, V, (N,), generator=gd, device=DEV)
    tg[::17] = -100
    with torch.enable_grad():
        lg = logits.clone().requires_grad_(True)
        loss = K.cross_entropy(lg, tg)
        loss.backward()
    lc, tc = logits.float().cpu(), tg.cpu()
    ref = O.cross_entropy(lc, tc)
    assert abs(float(loss) - float(ref)) <= 1e-4 * abs(float(ref)), (float(loss), float(ref))
    n_valid = int((tc != -100).sum())
    rows = [0, 1, 17, 1000, 4095]
    sm = torch.softmax(lc[rows], dim=-1)
    for j, r in enumerate(rows):
        want = torch.zeros(V) if int(tc[r]) == -100 else sm[j].clone()
        if int(tc[r]) != -100:
            want[int(tc[r])] -= 1.0
        assert_grad_close(lg.grad[r], want / n_valid, f"ce grad row {r}")
    twice_equal(lambda: (K.cross_entropy(logits, tg).reshape(1),))


# ------------------------------------------------------------------ norms, softmax, elementwise
def test_rmsnorm_backward_reference_shape_fp32():
    x, w, dy = rnd(4, 256, seed=20), rnd(256, seed=21), rnd(4, 256, seed=22)
    _, (gx, gw) = run_grads(lambda a, b: K.rmsnorm(a, b, 1e-6), [x, w], dy)
    _, (rx, rw) = ref_grads(lambda a, b: O.rmsnorm(a, b, 1e-6), [x, w], dy)
    assert_close(gx, rx, atol=1e-4, what="rmsnorm dx")
    assert_close(gw, rw, atol=1e-4, what="rmsnorm dw")


@pytest.mark.parametrize("rows,cols", [(512, 4096), (1000, 128), (33, 2048)])
def test_rmsnorm_backward_bf16(rows, cols):
    x, w, dy = rnd(rows, cols, seed=23).bfloat16(), (1 + 0.1 * rnd(cols, seed=24)).bfloat16(), rnd(rows, cols, seed=25)
    _, (gx, gw) = run_grads(lambda a, b: K.rmsnorm(a, b, 1e-6), [x, w], dy.bfloat16())
    _, (rx, rw) = ref_grads(lambda a, b: O.rmsnorm(a, b, 1e-6), [x, w], dy.bfloat16())
    assert_grad_close(gx, rx, "rmsnorm dx bf16")
    assert_grad_close(gw, rw, "rmsnorm dw bf16")
    twice_equal(lambda: run_grads(lambda a, b: K.rmsnorm(a, b, 1e-6), [x, w], dy.bfloat16())[1])


@pytest.mark.parametrize("rows,cols,dtype", [(4, 256, torch.float32), (3136, 1152, torch.bfloat16)])
def test_layernorm_backward(rows, cols, dtype):
    x, dy = rnd(rows, cols, seed=26, dtype=dtype), rnd(rows, cols, seed=29, dtype=dtype)
    w, b = (1 + 0.1 * rnd(cols, seed=27)).to(dtype), (0.1 * rnd(cols, seed=28)).to(dtype)
    _, (gx, gw, gb) = run_grads(lambda a, c, d: K.layernorm(a, c, d, 1e-6), [x, w, b], dy)
    _, (rx, rw, rb) = ref_grads(lambda a, c, d: O.layernorm(a, c, d, 1e-6), [x, w, b], dy)
    if dtype == torch.float32:
        for a, r, n in ((gx, rx, "dx"), (gw, rw, "dw"), (gb, rb, "db")):
            assert_close(a, r, atol=1e-4, what=f"layernorm {n}")
    else:
        for a, r, n in ((gx, rx, "dx"), (gw, rw, "dw"), (gb, rb, "db")):
            assert_grad_close(a, r, f"layernorm {n} bf16")


@pytest.mark.parametrize("rows,cols,dtype", [(8, 256, torch.float32), (4096, 128, torch.bfloat16)])
def test_softmax_backward(rows, cols, dtype):
    x, dy = rnd(rows, cols, seed=30, dtype=dtype), rnd(rows, cols, seed=31, dtype=dtype)
    _, (gx,) = run_grads(K.softmax, [x], dy)
    _, (rx,) = ref_grads(O.softmax, [x], dy)
    if dtype == torch.float32:
        assert_close(gx, rx, atol=1e-5, what="softmax dx")
    else:
        assert_grad_close(gx, rx, "softmax dx bf16")


@pytest.mark.parametrize("n,dtype", [((8, 128), torch.float32), ((64, 12288), torch.bfloat16)])
def test_swiglu_and_gelu_backward(n, dtype):
    a, b, dy = rnd(*n, seed=32, dtype=dtype), rnd(*n, seed=33, dtype=dtype), rnd(*n, seed=34, dtype=dtype)
    _, (ga, gb) = run_grads(K.swiglu, [a, b], dy)
    _, (ra, rb) = ref_grads(O.swiglu, [a, b], dy)
    _, (gg,) = run_grads(K.gelu_tanh, [a], dy)
    _, (rg,) = ref_grads(O.gelu_tanh, [a], dy)
    _, (g1, g2) = run_grads(K.residual_add, [a, b], dy)
    if dtype == torch.float32:
        assert_close(ga, ra, atol=1e-4, what="swiglu dgate")
        assert_close(gb, rb, atol=1e-4, what="swiglu dup")
        assert_close(gg, rg, atol=1e-4, what="gelu dx")
    else:
        assert_grad_close(ga, ra, "swiglu dgate bf16")
        assert_grad_close(gb, rb, "swiglu dup bf16")
        assert_grad_close(gg, rg, "gelu dx bf16")
    assert torch.equal(g1, dy.to(DEV)) and torch.equal(g2, dy.to(DEV))


# ------------------------------------------------------------------ GEMMs
def test_matmul_backward_reference_shape_fp32():
    x, w, b, dy = rnd(8, 64, seed=40), rnd(32, 64, seed=41), rnd(32, seed=42), rnd(8, 32, seed=43)
    _, (gx, gw, gb) = run_grads(K.matmul, [x, w, b], dy)
    _, (rx, rw, rb) = ref_grads(O.linear, [x, w, b], dy)
    for a, r, n in ((gx, rx, "dx"), (gw, rw, "dw"), (gb, rb, "db")):
        assert_close(a, r, atol=1e-3, what=f"matmul {n}")


@pytest.mark.parametrize("shape", [(2, 256, 1024, 768), (1, 300, 520, 264), (1, 32, 4096, 4096)])
def test_matmul_backward_bf16(shape):
    B, S, K_, N = shape
    x, w = rnd(B, S, K_, seed=44).bfloat16(), rnd(N, K_, seed=45, std=0.02).bfloat16()
    b, dy = rnd(N, seed=46, std=0.02).bfloat16(), rnd(B, S, N, seed=47).bfloat16()
    _, (gx, gw, gb) = run_grads(K.matmul, [x, w, b], dy)
    _, (rx, rw, rb) = ref_grads(O.linear, [x, w, b], dy)
    for a, r, n in ((gx, rx, "dx"), (gw, rw, "dw"), (gb, rb, "db")):
        assert_grad_close(a, r, f"matmul {n} bf16 {shape}")
    twice_equal(lambda: run_grads(K.matmul, [x, w, b], dy)[1])


def test_matmul_residual_gradient_passes_through():
    x, w, r, dy = rnd(40, 64, seed=48), rnd(24, 64, seed=49), rnd(40, 24, seed=50), rnd(40, 24, seed=51)
    _, (gx, gw, gr) = run_grads(lambda a, c, d: K.matmul(a, c, residual=d), [x, w, r], dy)
    _, (rx, rw, rr) = ref_grads(lambda a, c, d: O.linear(a, c) + d, [x, w, r], dy)
    assert_close(gx, rx, atol=1e-3, what="dx")
    assert_close(gw, rw, atol=1e-3, what="dw")
    assert torch.equal(gr.cpu(), dy)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_batched_gemm_backward(dtype):
    x, w, dy = rnd(4, 40, 64, seed=52, dtype=dtype), rnd(4, 48, 64, seed=53, dtype=dtype), rnd(4, 40, 48, seed=54,
                                                                                              dtype=dtype)
    _, (gx, gw) = run_grads(K.cuda_batched_gemm, [x, w], dy)
    _, (rx, rw) = ref_grads(O.batched_gemm, [x, w], dy)
    if dtype == torch.float32:
        assert_close(gx, rx, atol=1e-3, what="bgemm dx")
        assert_close(gw, rw, atol=1e-3, what="bgemm dw")
    else:
        assert_grad_close(gx, rx, "bgemm dx bf16")
        assert_grad_close(gw, rw, "bgemm dw bf16")


# ------------------------------------------------------------------ attention
def _fa(groups, causal, scale):
    return lambda q, k, v: K.flash_attention(q, k, v, scale, causal, groups)


def _fa_ref(groups, causal, scale):
    return lambda q, k, v: O.flash_attention(q, k, v, scale, causal, groups)


@pytest.mark.parametrize("Hq,Hkv,causal", [(4, 4, True), (4, 4, False), (8, 2, True)])
def test_flash_attention_backward_reference_shapes_fp32(Hq, Hkv, causal):
    q, k, v = rnd(2, Hq, 16, 32, seed=60), rnd(2, Hkv, 16, 32, seed=61), rnd(2, Hkv, 16, 32, seed=62)
    dy = rnd(2, Hq, 16, 32, seed=63)
    s = 32 ** -0.5
    _, (gq, gk, gv) = run_grads(_fa(Hq // Hkv, causal, s), [q, k, v], dy)
    _, (rq, rk, rv) = ref_grads(_fa_ref(Hq // Hkv, causal, s), [q, k, v], dy)
    for a, r, n in ((gq, rq, "dq"), (gk, rk, "dk"), (gv, rv, "dv")):
        assert_close(a, r, atol=5e-3, what=f"flash {n}")


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,causal", [
    (1, 8, 2, 300, 300, 128, True),    # text GQA, ragged key tiles
    (2, 4, 4, 100, 100, 72, False),    # vision head dim, non-causal
    (1, 8, 1, 130, 130, 64, True),     # groups 8
    (1, 4, 2, 5, 77, 128, False),      # Sq != Sk
])
def test_flash_attention_backward_bf16(B, Hq, Hkv, Sq, Sk, D, causal):
    q, k, v = (rnd(B, Hq, Sq, D, seed=64).bfloat16(), rnd(B, Hkv, Sk, D, seed=65).bfloat16(),
               rnd(B, Hkv, Sk, D, seed=66).bfloat16())
    dy = rnd(B, Hq, Sq, D, seed=67).bfloat16()
    s = D ** -0.5
    _, (gq, gk, gv) = run_grads(_fa(Hq // Hkv, causal, s), [q, k, v], dy)
    _, (rq, rk, rv) = ref_grads(_fa_ref(Hq // Hkv, causal, s), [q, k, v], dy)
    for a, r, n in ((gq, rq, "dq"), (gk, rk, "dk"), (gv, rv, "dv")):
        assert_grad_close(a, r, f"flash {n} bf16 D={D}")
    twice_equal(lambda: run_grads(_fa(Hq // Hkv, causal, s), [q, k, v], dy)[1])


# ------------------------------------------------------------------ embedding, rotary, routing
@pytest.mark.parametrize("dtype,padding_idx", [(torch.float32, None), (torch.bfloat16, 3)])
def test_embedding_backward(dtype, padding_idx):
    w = rnd(100, 64, seed=70, dtype=dtype)
    ids = torch.randint(0, 100, (4, 16), generator=torch.Generator().manual_seed(71))
    ids[0, :4] = 3  # repeated ids (and the padding row) accumulate
    dy = rnd(4, 16, 64, seed=72, dtype=dtype)
    with torch.enable_grad():
        wd = w.detach().to(DEV).clone().requires_grad_(True)
        K.embedding(ids.to(DEV), wd, padding_idx).backward(dy.to(DEV))
        wr = w.detach().float().clone().requires_grad_(True)
        F.embedding(ids, wr, padding_idx=padding_idx).backward(dy.float())
    if dtype == torch.float32:
        assert_close(wd.grad, wr.grad, atol=1e-5, what="embedding dw")
    else:
        assert_grad_close(wd.grad, wr.grad, "embedding dw bf16")


def test_rope_and_mrope_backward():
    B, H, S, D = 2, 4, 50, 128
    x, dy = rnd(B, H, S, D, seed=73), rnd(B, H, S, D, seed=74)
    pos = torch.arange(S).view(1, 1, S).expand(3, B, S)
    cos3, sin3 = O.mrope_cos_sin(pos, D, 5e6)
    _, (gx,) = run_grads(lambda t: K.apply_mrope(t, cos3.to(DEV), sin3.to(DEV), [24, 20, 20]), [x], dy)
    _, (rx,) = ref_grads(lambda t: O.apply_mrope(t, cos3, sin3, [24, 20, 20]), [x], dy)
    assert_close(gx, rx, atol=1e-4, what="mrope dx")
    cos, sin = cos3[0, 0, :, :72], sin3[0, 0, :, :72]
    x2, dy2 = rnd(B, H, S, 72, seed=75), rnd(B, H, S, 72, seed=76)
    _, (gx,) = run_grads(lambda t: K.apply_rope(t, cos.to(DEV), sin.to(DEV)), [x2], dy2)
    _, (rx,) = ref_grads(lambda t: O.apply_rope(t, cos, sin), [x2], dy2)
    assert_close(gx, rx, atol=1e-4, what="rope dx")


def test_topk_and_index_add_backward():
    x = rnd(64, 128, seed=77)
    gv = rnd(64, 8, seed=78)
    with torch.enable_grad():
        xd = x.to(DEV).requires_grad_(True)
        vals, idx = K.cuda_topk(xd, 8)
        vals.backward(gv.to(DEV))
    want = torch.zeros(64, 128).scatter_(-1, idx.cpu(), gv)
    assert torch.equal(xd.grad.cpu(), want)
    tgt, src = rnd(10, 16, seed=79), rnd(24, 16, seed=80)
    index = torch.randint(0, 10, (24,), generator=torch.Generator().manual_seed(81))
    dy = rnd(10, 16, seed=82)
    with torch.enable_grad():
        td, sd = tgt.to(DEV).requires_grad_(True), src.to(DEV).requires_grad_(True)
        out = K.cuda_index_add(td, sd, index.to(DEV))
        out.backward(dy.to(DEV))
    assert_close(out, tgt.index_add(0, index, src), atol=1e-5, what="index_add (autograd form)")
    assert torch.equal(td.grad.cpu(), dy) and torch.equal(sd.grad.cpu(), dy[index])
    assert torch.equal(td.detach().cpu(), tgt), "the autograd form leaves target unchanged"


def test_ops_without_backward_still_refuse_grad():
    x = rnd(8, 64, seed=83).to(DEV).requires_grad_(True)
    w = rnd(16, 64, seed=84).to(DEV)
    with torch.enable_grad(), pytest.raises(NotImplementedError):
        K.matmul_swiglu(x, w, w)


# ------------------------------------------------------------------ module-level training
def _module_grads(layer, fwd, x, dy):
    layer.requires_grad_(True)
    with torch.enable_grad():
        xd = x.detach().to(DEV).clone().requires_grad_(True)
        y = fwd(layer, xd)
        y.backward(dy.to(DEV).to(y.dtype))
    grads = {n: p.grad.float().cpu() for n, p in layer.named_parameters()}
    return y.detach().float().cpu(), xd.grad.float().cpu(), grads


def _oracle_grads(fn, p_dev, x, dy):
    p = {n: t.detach().float().cpu().requires_grad_(True) for n, t in p_dev.items()}
    with torch.enable_grad():
        xc = x.detach().float().cpu().clone().requires_grad_(True)
        y = fn(xc, p)
        y.backward(dy.float())
    return y.detach(), xc.grad, {n: t.grad for n, t in p.items()}


def _check_grads(got, ref, what, dtype):
    y, gx, gp = got
    ry, rgx, rgp = ref
    # bf16: a layer's backward rounds each of its ~20 intermediates to bf16, so its gradients carry
    # that accumulated rounding: max error within 5% of the largest |reference|, mean within 1.5%
    close = (lambda a, b, n: assert_close(a, b, atol=2e-3 * max(1.0, float(b.abs().max())), what=n)) \
        if dtype == torch.float32 else (lambda a, b, n: assert_grad_close(a, b, n, max_rel=5e-2, mean_rel=1.5e-2))
    close(y, ry, f"{what} output")
    close(gx, rgx, f"{what} d input")
    assert set(gp) == set(rgp)
    for n in gp:
        close(gp[n], rgp[n], f"{what} d {n}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_text_decoder_layer_trains_like_the_oracle(dtype):
    from oracle import layers as L
    from qwen3_5_vl_cuda_custom_amd import workloads as W
    cfg = W.C1
    layer = W.make_text_layer(cfg, dtype, DEV, seed=3)
    x, pos = W.text_inputs(cfg, 1, 128, dtype, DEV, seed=3)
    dy = rnd(1, 128, cfg.hidden, seed=90).to(dtype)
    bind = W.make_rope(cfg, DEV).bind(pos)
    got = _module_grads(layer, lambda m, t: m(t, bind)[0], x, dy)
    cos3, sin3 = O.mrope_cos_sin(pos.cpu(), cfg.head_dim, cfg.theta)
    kw = dict(num_heads=cfg.heads, num_kv_heads=cfg.kv_heads, head_dim=cfg.head_dim, eps=cfg.eps, cos_3d=cos3,
              sin_3d=sin3, mrope_section=list(cfg.mrope_section))
    ref = _oracle_grads(lambda t, p: L.text_decoder_layer(t, p, **kw)[0], dict(layer.named_parameters()), x, dy)
    _check_grads(got, ref, f"text layer {dtype}", dtype)


def test_moe_layer_trains_like_the_oracle():
    from oracle import layers as L
    from qwen3_5_vl_cuda_custom_amd.modules import CudaSparseMoE
    moe = CudaSparseMoE(hidden_size=128, moe_intermediate_size=48, num_experts=8, top_k=2).to(DEV)
    x, dy = rnd(1, 64, 128, seed=91), rnd(1, 64, 128, seed=92)
    got = _module_grads(moe, lambda m, t: m(t)[0], x, dy)
    ref = _oracle_grads(lambda t, p: L.sparse_moe(t, p, top_k=2)[0], dict(moe.named_parameters()), x, dy)
    _check_grads(got, ref, "moe layer", torch.float32)


def test_vision_block_trains_like_the_oracle():
    from oracle import layers as L
    from qwen3_5_vl_cuda_custom_amd.modules import CudaVisionBlock
    from qwen3_5_vl_cuda_custom_amd import workloads as W
    blk = CudaVisionBlock(288, 4, 400).to(DEV)
    W.init_normal_(blk, seed=5, std=0.05, include_bias=True)
    cos, sin = L.vision_rope_tables([(1, 8, 8)], 72, 1e4, 2)
    x, dy = rnd(2, 64, 288, seed=93), rnd(2, 64, 288, seed=94)
    got = _module_grads(blk, lambda m, t: m(t, cos.to(DEV), sin.to(DEV)), x, dy)
    ref = _oracle_grads(lambda t, p: L.vision_block(t, p, num_heads=4, cos=cos, sin=sin, eps=1e-6),
                        dict(blk.named_parameters()), x, dy)
    _check_grads(got, ref, "vision block", torch.float32)
