"""VisionMamba encoder (reference mlx_vision_mamba/vision_mamba.py:25-228).

Same interface as the reference: (B, H, W, C) / (B, D, H, W, C) /
(B, T, D, H, W, C) channel-last inputs, or pre-embedded (B, N, E) tokens,
mapped to (B, N, E) token features; K = 4 / 6 / 8 scan directions for 2D /
3D / 4D grids; optional ``patch_indices`` for a subset of tokens.
``scan_mode`` is passed down to every block.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn

from .mamba_block import MultiDirectionalMambaBlock
from .norm import layer_norm
from .vit import PatchEmbed, PatchEmbed3D, embed_3d


class PatchEmbed4D(nn.Module):
    """(B, T, D, H, W, C) -> (B, (T/tp)*(D/p)*(H/p)*(W/p), E): temporal
    patches folded into channels, then a 3D patch embedding per frame group
    (vision_mamba.py:25-94)."""

    def __init__(self, in_channels: int = 1, embed_dim: int = 384, patch_size: int = 16,
                 temporal_patch_size: int = 1):
        super().__init__()
        self.patch_size = patch_size
        self.temporal_patch_size = temporal_patch_size
        self.proj = nn.Conv3d(in_channels * temporal_patch_size, embed_dim,
                              kernel_size=patch_size, stride=patch_size, bias=True)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        bsz, T, Dd, H, W, C = x.shape
        tp = self.temporal_patch_size
        t_out = T // tp
        if tp > 1:                                                     # :75-81
            x = x[:, :t_out * tp].reshape(bsz, t_out, tp, Dd, H, W, C)
            x = x.permute(0, 1, 3, 4, 5, 2, 6).reshape(bsz, t_out, Dd, H, W, tp * C)
        x = x.reshape(bsz * t_out, Dd, H, W, -1)                       # :86
        out = embed_3d(x, self.proj, self.patch_size)                  # (B*T', Dp*Hp*Wp, E)
        return out.reshape(bsz, -1, out.shape[-1])                     # :93


class VisionMamba(nn.Module):
    """PatchEmbed -> [MultiDirectionalMambaBlock x depth] -> LayerNorm
    (vision_mamba.py:97-224)."""

    def __init__(self, img_size: int = 224, patch_size: int = 16, in_channels: int = 1,
                 embed_dim: int = 384, depth: int = 6, d_state: int = 16, d_conv: int = 4,
                 expand_factor: int = 2, input_dim: int = 2, temporal_patch_size: int = 1,
                 num_temporal_frames: int = 1, scan_mode: str = "sequential"):
        super().__init__()
        self.embed_dim = embed_dim
        self.input_dim = input_dim
        self.img_size = img_size
        self.patch_size = patch_size
        g = img_size // patch_size                                     # :148
        if input_dim == 2:
            self.grid_shape = (g, g)
            num_directions = 4
            self.patch_embed = PatchEmbed(in_channels, embed_dim, patch_size)
        elif input_dim == 3:
            self.grid_shape = (g, g, g)
            num_directions = 6
            self.patch_embed = PatchEmbed3D(in_channels, embed_dim, patch_size)
        elif input_dim == 4:
            tg = num_temporal_frames // temporal_patch_size
            self.grid_shape = (tg, g, g, g)
            num_directions = 8
            self.patch_embed = PatchEmbed4D(in_channels, embed_dim, patch_size,
                                            temporal_patch_size)
        else:
            raise ValueError(f"input_dim must be 2, 3, or 4, got {input_dim}")
        self.num_patches = math.prod(self.grid_shape)
        self.num_directions = num_directions
        self.pos_embed = nn.Parameter(torch.randn(1, self.num_patches, embed_dim)
                                      / math.sqrt(embed_dim))          # :178-181
        self.blocks = nn.ModuleList([
            MultiDirectionalMambaBlock(embed_dim, d_state, d_conv, expand_factor,
                                       num_directions=num_directions,
                                       grid_shape=self.grid_shape, scan_mode=scan_mode)
            for _ in range(depth)])
        self.norm = nn.LayerNorm(embed_dim)

    def forward(self, x: torch.Tensor, patch_indices: torch.Tensor = None) -> torch.Tensor:
        if x.ndim != 3:                                                # :211-212
            x = self.patch_embed(x)
        if patch_indices is not None:                                  # :214-218
            x = x + self.pos_embed[:, patch_indices, :]
        else:
            x = x + self.pos_embed
        for block in self.blocks:                                      # :220-221
            x = block(x)
        return layer_norm(x, self.norm)                                # :223

    def embed_patches(self, images: torch.Tensor) -> torch.Tensor:
        return self.patch_embed(images)                                # :226-228
