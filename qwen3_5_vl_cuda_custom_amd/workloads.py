"""Synthetic workloads of the benchmark configurations (seeded weights and inputs).

C1  tiny dense decoder layer, fp32: B1 S128 h256, 4q/2kv heads x 64, I 688, mrope [12,10,10]
C2  Qwen3-VL-8B-shape dense decoder layer, bf16 prefill: h4096, 32q/8kv x 128, I 12288, [24,20,20], S in {1024, 4096, 16384}
C3  the C2 layer in bf16 decode: B32, one new token each, KV cache lengths U[1024, 8192]
C4  Qwen3-VL-30B-A3B-shape MoE decoder layer, bf16: 4096 tokens, h2048, 32q/4kv x 128, 128 experts top-8, I_e 768
C5  Qwen3-VL vision block, bf16: 4 images of [2, 3, 448, 448] -> 4 x 784 patches, h1152, 16 heads x 72, I 4304

Weights are N(0, 0.02) (norm weights keep their module default of ones; vision
biases N(0, 0.02)); text inputs N(0, 1); pixels U(-1, 1); mRoPE theta 5e6 with
text positions 0..S-1 on all three axes.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .modules import CudaTextDecoderLayer, CudaVisionBlock, CudaVisionPatchEmbed, StaticKVCache, TextMRoPE


@dataclass(frozen=True)
class TextLayerConfig:
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    eps: float = 1e-6
    theta: float = 5e6
    mrope_section: tuple[int, int, int] = (24, 20, 20)
    use_moe: bool = False
    num_experts: int = 0
    top_k: int = 0
    moe_intermediate: int = 0

    def gemm_flops_per_token(self) -> int:
        """2 * (q + k + v + o + MLP) weight elements per token."""
        h, d = self.hidden, self.head_dim
        attn = h * d * (2 * self.heads + 2 * self.kv_heads)
        mlp = (3 * h * self.moe_intermediate * self.top_k + h * self.num_experts) if self.use_moe \
            else 3 * h * self.intermediate
        return 2 * (attn + mlp)

    def causal_attn_flops(self, seq: int, batch: int = 1) -> int:
        """QK^T + PV over the causal triangle: 4 * D * Hq * S(S+1)/2 per sequence."""
        return 4 * self.head_dim * self.heads * seq * (seq + 1) // 2 * batch


C1 = TextLayerConfig(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=688, mrope_section=(12, 10, 10))
C2 = TextLayerConfig(hidden=4096, heads=32, kv_heads=8, head_dim=128, intermediate=12288)
C4 = TextLayerConfig(hidden=2048, heads=32, kv_heads=4, head_dim=128, intermediate=0, use_moe=True,
                     num_experts=128, top_k=8, moe_intermediate=768)


@dataclass(frozen=True)
class VisionConfig:
    hidden: int = 1152
    heads: int = 16
    intermediate: int = 4304
    patch: int = 16
    temporal: int = 2
    channels: int = 3
    merge: int = 2
    theta: float = 1e4
    eps: float = 1e-6
    images: int = 4
    image_hw: tuple[int, int] = (448, 448)
    frames: int = 2

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @property
    def grid(self) -> tuple[int, int, int]:
        return (self.frames // self.temporal, self.image_hw[0] // self.patch, self.image_hw[1] // self.patch)

    @property
    def patches_per_image(self) -> int:
        t, h, w = self.grid
        return t * h * w

    def flops(self) -> int:
        """Patch-embed GEMM + one block (qkv, proj, fc1, fc2, full attention per image)."""
        n = self.images * self.patches_per_image
        k_in = self.channels * self.temporal * self.patch * self.patch
        h = self.hidden
        gemm = 2 * n * (k_in * h + 4 * h * h + 2 * h * self.intermediate)
        attn = 4 * self.head_dim * self.heads * self.patches_per_image ** 2 * self.images
        return gemm + attn


C5 = VisionConfig()


def _gen(device: torch.device | str, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


@torch.no_grad()
def init_normal_(module: torch.nn.Module, seed: int, std: float = 0.02, include_bias: bool = False) -> None:
    """Every weight matrix (and, optionally, bias) ~ N(0, std); 1-D norm weights keep their default."""
    dev = next(module.parameters()).device
    g = _gen(dev, seed)
    for name, p in module.named_parameters():
        is_norm = "norm" in name.split(".")[-2] if "." in name else False
        if p.dim() >= 2 and not is_norm:
            p.normal_(0.0, std, generator=g)
        elif include_bias and name.endswith("bias") and not is_norm:
            p.normal_(0.0, std, generator=g)


def make_text_layer(cfg: TextLayerConfig, dtype=torch.bfloat16, device="cuda", seed: int = 0) -> CudaTextDecoderLayer:
    layer = CudaTextDecoderLayer(cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.intermediate, cfg.eps,
                                 use_moe=cfg.use_moe, num_experts=cfg.num_experts, top_k=cfg.top_k,
                                 moe_intermediate_size=cfg.moe_intermediate)
    layer = layer.to(device=device, dtype=dtype)
    init_normal_(layer, seed)
    return layer.eval().requires_grad_(False)


def make_rope(cfg: TextLayerConfig, device="cuda") -> TextMRoPE:
    return TextMRoPE(cfg.head_dim, theta=cfg.theta, mrope_section=list(cfg.mrope_section)).to(device)


def text_inputs(cfg: TextLayerConfig, batch: int, seq: int, dtype=torch.bfloat16, device="cuda", seed: int = 0):
    """x (B, S, h) ~ N(0, 1) and text positions (3, B, S) = 0..S-1 on every axis."""
    g = _gen(device, seed + 1)
    x = torch.randn(batch, seq, cfg.hidden, generator=g, device=device, dtype=torch.float32).to(dtype)
    pos = torch.arange(seq, device=device).view(1, 1, seq).expand(3, batch, seq).contiguous()
    return x, pos


@dataclass
class DecodeCase:
    layer: CudaTextDecoderLayer
    rope: TextMRoPE
    cache: StaticKVCache
    x: torch.Tensor
    positions: torch.Tensor
    lens: torch.Tensor = field(default_factory=lambda: torch.zeros(0))


def decode_lengths(batch: int = 32, seed: int = 0) -> torch.Tensor:
    """Per-sequence KV lengths U[1024, 8192] (CPU generator, so identical on every machine)."""
    return torch.randint(1024, 8193, (batch,), generator=torch.Generator().manual_seed(seed))


@torch.no_grad()
def make_decode_case(cfg: TextLayerConfig = C2, batch: int = 32, capacity: int = 8193, device="cuda",
                     seed: int = 0, layer: CudaTextDecoderLayer | None = None) -> DecodeCase:
    """C3: one new token per sequence, cache rows [0, L_b) filled N(0,1), new token written at row L_b."""
    layer = layer if layer is not None else make_text_layer(cfg, torch.bfloat16, device, seed)
    lens = decode_lengths(batch, seed)
    cache = StaticKVCache(batch, cfg.kv_heads, capacity, cfg.head_dim, dtype=torch.bfloat16, device=device,
                          lens=lens)
    g = _gen(device, seed + 2)
    cache.k.normal_(0.0, 1.0, generator=g)
    cache.v.normal_(0.0, 1.0, generator=g)
    x = torch.randn(batch, 1, cfg.hidden, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    pos = lens.to(device).view(1, batch, 1).expand(3, batch, 1).contiguous()
    return DecodeCase(layer, make_rope(cfg, device), cache, x, pos, lens)


def make_vision_block(cfg: VisionConfig = C5, dtype=torch.bfloat16, device="cuda", seed: int = 0) -> CudaVisionBlock:
    blk = CudaVisionBlock(cfg.hidden, cfg.heads, cfg.intermediate, eps=cfg.eps).to(device=device, dtype=dtype)
    init_normal_(blk, seed, include_bias=True)
    return blk.eval().requires_grad_(False)


def make_patch_embed(cfg: VisionConfig = C5, dtype=torch.bfloat16, device="cuda", seed: int = 0):
    pe = CudaVisionPatchEmbed(cfg.channels, cfg.hidden, cfg.patch, cfg.temporal).to(device=device, dtype=dtype)
    init_normal_(pe, seed + 7, include_bias=True)
    return pe.eval().requires_grad_(False)


def patchify(pixels: torch.Tensor, cfg: VisionConfig = C5) -> torch.Tensor:
    """(images, frames, C, H, W) -> (images * patches, C*T*P*P) in the merge-block order.

    Patches of one image are ordered (t, h/m, w/m, m_h, m_w) and each patch is
    flattened as (C, T, P, P), the layout the Qwen2/3-VL image processor emits.
    """
    n, f, c, hh, ww = pixels.shape
    t, p, m = cfg.temporal, cfg.patch, cfg.merge
    gt, gh, gw = f // t, hh // p, ww // p
    x = pixels.reshape(n, gt, t, c, gh // m, m, p, gw // m, m, p)
    # -> (n, gt, gh/m, gw/m, m_h, m_w, c, t, p_h, p_w)
    x = x.permute(0, 1, 4, 7, 5, 8, 3, 2, 6, 9)
    return x.reshape(n * gt * gh * gw, c * t * p * p)


def vision_inputs(cfg: VisionConfig = C5, dtype=torch.bfloat16, device="cuda", seed: int = 0) -> torch.Tensor:
    """Pixels (images, frames, 3, H, W) ~ U(-1, 1), patchified to (N, C*T*P*P)."""
    g = _gen(device, seed + 3)
    px = torch.rand(cfg.images, cfg.frames, cfg.channels, *cfg.image_hw, generator=g, device=device) * 2 - 1
    return patchify(px, cfg).to(dtype)


def vision_rope_cos_sin(cfg: VisionConfig = C5, device="cuda"):
    """cos/sin (patches_per_image, head_dim) fp32 for one image's (t, h, w) grid.

    The vision tower's 2D rope (merge-block (row, col) coordinates, inv_freq
    over head_dim/2, emb = cat(rot, rot)); every image of C5 has the same grid,
    so one table serves the whole batch.
    """
    hd = cfg.head_dim
    rot_dim = hd // 2
    inv_freq = 1.0 / (cfg.theta ** (torch.arange(0, rot_dim, 2, dtype=torch.float32, device=device) / rot_dim))
    t, h, w = cfg.grid
    m = cfg.merge
    rows = (torch.arange(h // m, device=device)[:, None, None, None] * m
            + torch.arange(m, device=device)[None, None, :, None]).expand(h // m, w // m, m, m).reshape(-1)
    cols = (torch.arange(w // m, device=device)[None, :, None, None] * m
            + torch.arange(m, device=device)[None, None, None, :]).expand(h // m, w // m, m, m).reshape(-1)
    rows, cols = rows.repeat(t), cols.repeat(t)
    rot = torch.cat([rows.float()[:, None] * inv_freq, cols.float()[:, None] * inv_freq], dim=-1)
    emb = torch.cat([rot, rot], dim=-1)
    return emb.cos(), emb.sin()
