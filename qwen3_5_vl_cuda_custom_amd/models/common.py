"""CudaVisionTower (reference models/common.py:24-246): patch embed, interpolated position
embedding, 2D rotary, vision blocks, deepstack mergers and the final merger.

Every step runs on the GPU kernels: the position-embedding interpolation and
the rotary tables are computed by kernels from the images' grids (the
reference builds them with host loops and small torch ops), and each image
frame attends only within itself through packed variable-length attention
(`cu_seqlens`, as HF's Qwen3VLVisionModel does; the reference runs the blocks
over one concatenated sequence, models/common.py:198, which makes images
attend to each other).
"""
from __future__ import annotations

import torch
from torch import nn

from ..configs import VisionConfig
from ..kernels import vision_pos_embed, vision_rope_tables
from ..modules import CudaEmbedding, CudaVisionBlock, CudaVisionPatchEmbed, CudaVisionPatchMerger
from ..modules.rotary import _FP32Freqs, rotary_inv_freq


class _PosEmbedWrap(nn.Module):
    """The learned (num_positions, hidden) grid under the reference's `pos_embed.emb.weight` key."""

    def __init__(self, num_embeddings: int, embedding_dim: int) -> None:
        super().__init__()
        self.emb = CudaEmbedding(num_embeddings, embedding_dim)

    @property
    def weight(self) -> torch.Tensor:
        return self.emb.weight

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return self.emb(ids)


def grid_list(grid_thw) -> list[tuple[int, int, int]]:
    """(t, h, w) per image from an (n, 3) tensor or a sequence of triples (read on the host)."""
    rows = grid_thw.tolist() if torch.is_tensor(grid_thw) else grid_thw
    return [tuple(int(v) for v in r) for r in rows]


def frame_seqlens(grid_thw, device) -> tuple[torch.Tensor, int]:
    """cu_seqlens over the frames (each frame of each image is one h*w-token sequence) and the longest."""
    lens = [h * w for t, h, w in grid_list(grid_thw) for _ in range(t)]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    return torch.tensor(cu, dtype=torch.int32).to(device), max(lens)


class CudaVisionTower(_FP32Freqs):
    """forward(hidden_states (N, C*T*P*P), grid_thw (n_images, 3)) ->
    (pooler_output (N / merge^2, out_hidden), last_hidden_state (N, hidden),
    deepstack_features [(N / merge^2, out_hidden)] per deepstack layer)."""

    def __init__(self, cfg: VisionConfig) -> None:
        super().__init__()
        self.cfg = cfg
        self.spatial_merge_size = cfg.spatial_merge_size
        self.patch_size = cfg.patch_size
        self.num_grid_per_side = int(cfg.num_position_embeddings ** 0.5)
        self.patch_embed = CudaVisionPatchEmbed(in_channels=cfg.in_channels, hidden_size=cfg.hidden_size,
                                                patch_size=cfg.patch_size,
                                                temporal_patch_size=cfg.temporal_patch_size)
        self.pos_embed = _PosEmbedWrap(cfg.num_position_embeddings, cfg.hidden_size)
        head_dim = cfg.hidden_size // cfg.num_heads
        self.head_dim = head_dim
        self.rotary_dim = head_dim // 2
        self._freq_dim, self._freq_theta = self.rotary_dim, cfg.rope_theta
        self.register_buffer("inv_freq", rotary_inv_freq(self.rotary_dim, cfg.rope_theta), persistent=False)
        self.blocks = nn.ModuleList([CudaVisionBlock(cfg.hidden_size, cfg.num_heads, cfg.intermediate_size,
                                                     eps=cfg.rms_norm_eps) for _ in range(cfg.num_layers)])
        self.merger = CudaVisionPatchMerger(cfg.hidden_size, cfg.out_hidden_size, cfg.spatial_merge_size,
                                            use_postshuffle_norm=False)
        self.deepstack_mergers = nn.ModuleList([
            CudaVisionPatchMerger(cfg.hidden_size, cfg.out_hidden_size, cfg.spatial_merge_size,
                                  use_postshuffle_norm=True) for _ in cfg.deepstack_layers])

    def rotary_tables(self, grid_thw) -> tuple[torch.Tensor, torch.Tensor]:
        """cos, sin (N, head_dim) fp32 of every patch (the reference's _rot_pos_emb + cat + cos/sin)."""
        return vision_rope_tables(grid_list(grid_thw), self.spatial_merge_size, self.inv_freq, self.head_dim)

    def forward(self, hidden_states: torch.Tensor, grid_thw):
        grids = grid_list(grid_thw)
        x = self.patch_embed(hidden_states)
        x = vision_pos_embed(x, self.pos_embed.weight, grids, self.spatial_merge_size, out=x)
        cos, sin = self.rotary_tables(grids)
        cu, max_len = frame_seqlens(grids, x.device)
        x = x.unsqueeze(0)
        where = {layer: i for i, layer in enumerate(self.cfg.deepstack_layers)}
        deepstack = []
        for i, block in enumerate(self.blocks):
            x = block(x, cos, sin, cu_seqlens=cu, max_seqlen=max_len)
            if i in where:
                deepstack.append(self.deepstack_mergers[where[i]](x[0]))
        last = x[0]
        return self.merger(last), last, deepstack
