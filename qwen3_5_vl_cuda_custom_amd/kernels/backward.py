"""Autograd for the functional ops: one torch.autograd.Function per op that has
one in the reference (kernels/{matmul,flash_attention,rmsnorm,layernorm,softmax,
swiglu,gelu_tanh,sigmoid_mul,residual_add,cross_entropy,embedding,mrope,rope,
moe_routing}.py), whose forward runs the op's HIP kernel and whose backward runs
the HIP backward kernels of libq3vl.so (train.hip, attention_bwd.hip). No
backward falls back to torch: a kernel that cannot run raises.

Every backward is deterministic (fixed-order reductions, no atomics), so the
same inputs give bitwise identical gradients run to run.
"""
from __future__ import annotations

import torch

from .. import _lib


def needs_grad(*tensors) -> bool:
    """True when autograd must record the op (grad mode on and an input requires grad)."""
    return torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)


def _c(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _dt(t: torch.Tensor) -> int:
    return _lib.dtype_code(t.dtype)


# ------------------------------------------------------------------ GEMMs
class MatmulFunction(torch.autograd.Function):
    """y = x·Wᵀ + b (+ residual). Reference: kernels/matmul.py:20-59, csrc/matmul_op.cu:151-233.
    dx = dy·W, dW = dyᵀ·x, db = Σ_rows dy, d(residual) = dy."""

    @staticmethod
    def forward(ctx, x, weight, bias, residual):
        from .matmul import matmul
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        ctx.has_residual = residual is not None
        return matmul(x, weight, bias, residual=residual)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        K, N = x.shape[-1], w.shape[0]
        x2 = _c(x.reshape(-1, K))
        dy2 = _c(dy.reshape(-1, N)).to(x.dtype)
        M = x2.shape[0]
        need_x, need_w, need_b, need_r = ctx.needs_input_grad
        gx = torch.empty((M, K), dtype=x.dtype, device=x.device) if need_x else None
        gw = torch.empty((N, K), dtype=w.dtype, device=w.device) if need_w else None
        gb = torch.empty((N,), dtype=w.dtype, device=w.device) if (need_b and ctx.has_bias) else None
        lib = _lib.lib()
        ws, nws = _lib.workspace(lib.q3_matmul_backward_workspace_bytes(M, N, K, _dt(x)), x.device)
        gneed = max(lib.q3_matmul_workspace_bytes(M, K, N, _dt(x), 0), lib.q3_matmul_workspace_bytes(N, K, M, _dt(x), 0))
        gws, gnws = _lib.gemm_workspace(gneed, x.device)
        _lib.call("q3_matmul_backward", x2.data_ptr(), _c(w).data_ptr(), dy2.data_ptr(), _lib.ptr(gx), _lib.ptr(gw),
                  _lib.ptr(gb), M, N, K, _dt(x), _lib.ptr(ws), nws, _lib.ptr(gws), gnws, _lib.stream())
        gr = dy if (need_r and ctx.has_residual) else None
        return (gx.view(x.shape) if gx is not None else None), gw, gb, gr


class BatchedGemmFunction(torch.autograd.Function):
    """y[e] = x[e]·w[e]ᵀ. Reference: kernels/moe_routing.py:131-181."""

    @staticmethod
    def forward(ctx, x, w):
        from .moe_routing import cuda_batched_gemm
        ctx.save_for_backward(x, w)
        return cuda_batched_gemm(x, w)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        E, M, K = x.shape
        N = w.shape[1]
        need_x, need_w = ctx.needs_input_grad
        gx = torch.empty_like(x, memory_format=torch.contiguous_format) if need_x else None
        gw = torch.empty_like(w, memory_format=torch.contiguous_format) if need_w else None
        ws, nws = _lib.workspace(_lib.lib().q3_batched_gemm_backward_workspace_bytes(E, M, N, K, _dt(x)), x.device)
        _lib.call("q3_batched_gemm_backward", _c(x).data_ptr(), _c(w).data_ptr(), _c(dy).to(x.dtype).data_ptr(),
                  _lib.ptr(gx), _lib.ptr(gw), E, M, N, K, _dt(x), _lib.ptr(ws), nws, _lib.stream())
        return gx, gw


# ------------------------------------------------------------------ attention
class FlashAttentionFunction(torch.autograd.Function):
    """Reference: kernels/flash_attention.py:21-78, csrc/flash_attention_op.cu:235-390."""

    @staticmethod
    def forward(ctx, q, k, v, scale, is_causal, num_kv_groups):
        from .flash_attention import flash_attention_lse
        q, k, v = _c(q), _c(k), _c(v)
        o, lse = flash_attention_lse(q, k, v, scale, is_causal, num_kv_groups)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale, ctx.is_causal = float(scale), bool(is_causal)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        B, Hq, Sq, D = q.shape
        Hkv, Sk = k.shape[1], k.shape[2]
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        ws, nws = _lib.workspace(_lib.lib().q3_flash_attention_backward_workspace_bytes(B, Hq, Sq), q.device)
        _lib.call("q3_flash_attention_backward", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                  lse.data_ptr(), _c(do).to(q.dtype).data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, Hq,
                  Hkv, Sq, Sk, D, ctx.scale, int(ctx.is_causal), _dt(q), _lib.ptr(ws), nws, _lib.stream())
        return dq, dk, dv, None, None, None


# ------------------------------------------------------------------ norms / softmax
class RMSNormFunction(torch.autograd.Function):
    """Reference: kernels/rmsnorm.py:35-63, csrc/rmsnorm_op.cu:63-130."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        from .norms import rmsnorm
        ctx.save_for_backward(x, weight)
        ctx.eps = float(eps)
        return rmsnorm(x, weight, eps)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        cols = x.shape[-1]
        rows = x.numel() // cols
        xc = _c(x)
        gx = torch.empty_like(xc)
        gw = torch.empty_like(w) if ctx.needs_input_grad[1] else None
        ws, nws = _lib.workspace(_lib.lib().q3_norm_backward_workspace_bytes(rows, cols), x.device)
        _lib.call("q3_rmsnorm_backward", xc.data_ptr(), _c(w).data_ptr(), _c(dy).to(x.dtype).data_ptr(), gx.data_ptr(),
                  _lib.ptr(gw), rows, cols, ctx.eps, _dt(x), _lib.ptr(ws), nws, _lib.stream())
        return gx, gw, None


class LayerNormFunction(torch.autograd.Function):
    """Reference: kernels/layernorm.py:17-52 (there through torch autograd)."""

    @staticmethod
    def forward(ctx, x, weight, bias, eps):
        from .norms import layernorm
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        ctx.eps = float(eps)
        return layernorm(x, weight, bias, eps)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        cols = x.shape[-1]
        rows = x.numel() // cols
        xc = _c(x)
        gx = torch.empty_like(xc)
        gw = torch.empty_like(w) if ctx.needs_input_grad[1] else None
        gb = torch.empty_like(w) if (ctx.has_bias and ctx.needs_input_grad[2]) else None
        ws, nws = _lib.workspace(_lib.lib().q3_norm_backward_workspace_bytes(rows, cols), x.device)
        _lib.call("q3_layernorm_backward", xc.data_ptr(), _c(w).data_ptr(), _c(dy).to(x.dtype).data_ptr(),
                  gx.data_ptr(), _lib.ptr(gw), _lib.ptr(gb), rows, cols, ctx.eps, _dt(x), _lib.ptr(ws), nws,
                  _lib.stream())
        return gx, gw, gb, None


class SoftmaxFunction(torch.autograd.Function):
    """Reference: kernels/softmax.py:12-37, csrc/softmax_op.cu:55-88."""

    @staticmethod
    def forward(ctx, x):
        from .norms import softmax
        out = softmax(x)
        ctx.save_for_backward(out)
        return out

    @staticmethod
    def backward(ctx, dy):
        (out,) = ctx.saved_tensors
        cols = out.shape[-1]
        gx = torch.empty_like(out)
        _lib.call("q3_softmax_backward", out.data_ptr(), _c(dy).to(out.dtype).data_ptr(), gx.data_ptr(),
                  out.numel() // cols, cols, _dt(out), _lib.stream())
        return gx


# ------------------------------------------------------------------ elementwise
class SwiGLUFunction(torch.autograd.Function):
    """Reference: kernels/swiglu.py:27-53, csrc/swiglu_op.cu:20-39."""

    @staticmethod
    def forward(ctx, gate, up):
        from .elementwise import swiglu
        ctx.save_for_backward(gate, up)
        return swiglu(gate, up)

    @staticmethod
    def backward(ctx, dy):
        gate, up = (_c(t) for t in ctx.saved_tensors)
        gg, gu = torch.empty_like(gate), torch.empty_like(up)
        _lib.call("q3_swiglu_backward", gate.data_ptr(), up.data_ptr(), _c(dy).to(gate.dtype).data_ptr(),
                  gg.data_ptr(), gu.data_ptr(), gate.numel(), _dt(gate), _lib.stream())
        return gg, gu


class GeluTanhFunction(torch.autograd.Function):
    """Reference: kernels/gelu_tanh.py:17-46, csrc/gelu_tanh_op.cu:20-36."""

    @staticmethod
    def forward(ctx, x):
        from .elementwise import gelu_tanh
        ctx.save_for_backward(x)
        return gelu_tanh(x)

    @staticmethod
    def backward(ctx, dy):
        (x,) = ctx.saved_tensors
        x = _c(x)
        gx = torch.empty_like(x)
        _lib.call("q3_gelu_tanh_backward", x.data_ptr(), _c(dy).to(x.dtype).data_ptr(), gx.data_ptr(), x.numel(),
                  _dt(x), _lib.stream())
        return gx


class SigmoidMulFunction(torch.autograd.Function):
    """Reference: kernels/sigmoid_mul.py:23-46, csrc/sigmoid_mul_op.cu:18-34."""

    @staticmethod
    def forward(ctx, x, gate):
        from .elementwise import sigmoid_mul
        ctx.save_for_backward(x, gate)
        return sigmoid_mul(x, gate)

    @staticmethod
    def backward(ctx, dy):
        x, gate = (_c(t) for t in ctx.saved_tensors)
        gx, gg = torch.empty_like(x), torch.empty_like(gate)
        _lib.call("q3_sigmoid_mul_backward", x.data_ptr(), gate.data_ptr(), _c(dy).to(x.dtype).data_ptr(),
                  gx.data_ptr(), gg.data_ptr(), x.numel(), _dt(x), _lib.stream())
        return gx, gg


class ResidualAddFunction(torch.autograd.Function):
    """Reference: kernels/residual_add.py:12-25: both inputs receive the output gradient."""

    @staticmethod
    def forward(ctx, a, b):
        from .elementwise import residual_add
        return residual_add(a, b)

    @staticmethod
    def backward(ctx, dy):
        return dy, dy


# ------------------------------------------------------------------ loss, embedding
class CrossEntropyFunction(torch.autograd.Function):
    """Reference: kernels/cross_entropy.py:17-49, csrc/cross_entropy_op.cu:66-116.
    The backward reads the loss gradient and the valid-target count on the device."""

    @staticmethod
    def forward(ctx, logits, targets, ignore_index):
        from .cross_entropy import cross_entropy_fwd
        logits, targets = _c(logits), _c(targets)
        loss, lse, n_valid = cross_entropy_fwd(logits, targets, ignore_index)
        ctx.save_for_backward(logits, targets, lse, n_valid)
        ctx.ignore_index = int(ignore_index)
        return loss

    @staticmethod
    def backward(ctx, dloss):
        logits, targets, lse, n_valid = ctx.saved_tensors
        N, V = logits.shape
        g = torch.empty_like(logits)
        dl = _c(dloss.reshape(1).to(torch.float32))
        _lib.call("q3_cross_entropy_backward", logits.data_ptr(), targets.data_ptr(), lse.data_ptr(), dl.data_ptr(),
                  n_valid.data_ptr(), g.data_ptr(), N, V, ctx.ignore_index, _dt(logits), _lib.stream())
        return g, None, None


class EmbeddingFunction(torch.autograd.Function):
    """Reference: kernels/embedding.py:13-58, csrc/embedding_op.cu:71-97: the weight gradient sums the
    output-gradient rows of each id (here the deterministic index_add, fp32 sums in token order,
    one rounding); the padding row gets none."""

    @staticmethod
    def forward(ctx, ids, weight, padding_idx):
        from .embedding import embedding
        ctx.save_for_backward(ids)
        ctx.shape = tuple(weight.shape)
        ctx.padding_idx = padding_idx
        return embedding(ids, weight, padding_idx)

    @staticmethod
    def backward(ctx, dy):
        from .moe_routing import cuda_index_add
        (ids,) = ctx.saved_tensors
        V, D = ctx.shape
        gw = torch.zeros((V, D), dtype=dy.dtype, device=dy.device)
        with torch.no_grad():
            cuda_index_add(gw, _c(dy.reshape(-1, D)), ids.reshape(-1).to(torch.int64))
        if ctx.padding_idx is not None:
            gw[ctx.padding_idx].zero_()
        return None, gw, None


# ------------------------------------------------------------------ rotary
class MRopeFunction(torch.autograd.Function):
    """Reference: kernels/mrope.py:53-77: the gradient is the rotation by -sin."""

    @staticmethod
    def forward(ctx, x, cos_3d, sin_3d, mrope_section):
        from .rotary import apply_mrope
        ctx.save_for_backward(cos_3d, sin_3d)
        ctx.section = list(mrope_section)
        return apply_mrope(x, cos_3d, sin_3d, mrope_section)

    @staticmethod
    def backward(ctx, dy):
        from .rotary import apply_mrope
        cos_3d, sin_3d = ctx.saved_tensors
        with torch.no_grad():
            return apply_mrope(_c(dy), cos_3d, -sin_3d, ctx.section), None, None, None


class RopeFunction(torch.autograd.Function):
    """Reference: kernels/rope.py:31-55."""

    @staticmethod
    def forward(ctx, x, cos, sin):
        from .rotary import apply_rope
        ctx.save_for_backward(cos, sin)
        return apply_rope(x, cos, sin)

    @staticmethod
    def backward(ctx, dy):
        from .rotary import apply_rope
        cos, sin = ctx.saved_tensors
        with torch.no_grad():
            return apply_rope(_c(dy), cos, -sin), None, None


# ------------------------------------------------------------------ MoE routing
class TopKFunction(torch.autograd.Function):
    """Reference: kernels/moe_routing.py:26-52: the value gradients go back to their columns."""

    @staticmethod
    def forward(ctx, x, k):
        from .moe_routing import cuda_topk
        vals, idx = cuda_topk(x, k)
        ctx.save_for_backward(idx)
        ctx.shape = tuple(x.shape)
        ctx.mark_non_differentiable(idx)
        return vals, idx

    @staticmethod
    def backward(ctx, gvals, gidx):
        (idx,) = ctx.saved_tensors
        cols = ctx.shape[-1]
        k = idx.shape[-1]
        gx = torch.empty(ctx.shape, dtype=gvals.dtype, device=gvals.device)
        _lib.call("q3_topk_backward", _c(gvals).data_ptr(), idx.data_ptr(), gx.data_ptr(), gx.numel() // cols, cols,
                  k, _dt(gx), _lib.stream())
        return gx, None


class IndexAddFunction(torch.autograd.Function):
    """Reference: kernels/moe_routing.py:72-100: under autograd the op returns a new tensor
    (target + the scattered sources); d target = dy, d source = dy[index]."""

    @staticmethod
    def forward(ctx, target, source, index):
        from .moe_routing import cuda_index_add
        ctx.save_for_backward(index)
        ctx.source_shape = tuple(source.shape)
        return cuda_index_add(target.clone(), source, index)

    @staticmethod
    def backward(ctx, dy):
        from .embedding import embedding
        (index,) = ctx.saved_tensors
        D = dy[0].numel()
        with torch.no_grad():
            gs = embedding(index.to(torch.int64), _c(dy.reshape(dy.shape[0], D)))
        return dy, gs.reshape(ctx.source_shape), None
