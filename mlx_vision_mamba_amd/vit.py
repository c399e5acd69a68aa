"""Patch embeddings (reference mlx_vision_mamba/vit.py:48-92).

Channel-last inputs as in the reference.  A patch embedding with kernel ==
stride is a per-patch linear map, so it is computed as one GEMM over the
unfolded patches (weights kept in torch's conv layout (E, C, p, p[, p])).
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F


class PatchEmbed(nn.Module):
    """(B, H, W, C) -> (B, (H/p)*(W/p), E), row-major over the patch grid
    (vit.py:48-67)."""

    def __init__(self, in_channels: int = 1, embed_dim: int = 384, patch_size: int = 16):
        super().__init__()
        self.patch_size = patch_size
        self.proj = nn.Conv2d(in_channels, embed_dim, kernel_size=patch_size, stride=patch_size,
                              bias=True)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        bsz, H, W, C = x.shape
        p = self.patch_size
        hp, wp = H // p, W // p
        x = x[:, :hp * p, :wp * p]
        cols = x.reshape(bsz, hp, p, wp, p, C).permute(0, 1, 3, 5, 2, 4).reshape(bsz, hp * wp, C * p * p)
        return F.linear(cols, self.proj.weight.reshape(self.proj.out_channels, -1), self.proj.bias)


class PatchEmbed3D(nn.Module):
    """(B, D, H, W, C) -> (B, (D/p)*(H/p)*(W/p), E), row-major over the
    patch grid (vit.py:70-92)."""

    def __init__(self, in_channels: int = 1, embed_dim: int = 384, patch_size: int = 16):
        super().__init__()
        self.patch_size = patch_size
        self.proj = nn.Conv3d(in_channels, embed_dim, kernel_size=patch_size, stride=patch_size,
                              bias=True)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return embed_3d(x, self.proj, self.patch_size)


def embed_3d(x: torch.Tensor, proj: nn.Conv3d, p: int) -> torch.Tensor:
    """Channel-last (B, D, H, W, C) volume -> (B, patches, E) with the
    weights of a kernel == stride Conv3d, as one GEMM."""
    bsz, Dd, H, W, C = x.shape
    dp, hp, wp = Dd // p, H // p, W // p
    x = x[:, :dp * p, :hp * p, :wp * p]
    cols = x.reshape(bsz, dp, p, hp, p, wp, p, C).permute(0, 1, 3, 5, 7, 2, 4, 6)
    cols = cols.reshape(bsz, dp * hp * wp, C * p * p * p)
    return F.linear(cols, proj.weight.reshape(proj.out_channels, -1), proj.bias)
