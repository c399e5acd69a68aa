"""Mamba blocks on MI355X (PyTorch modules over the HIP selective scan).

Mirrors the reference's module API (mlx_vision_mamba/mamba_block.py):
``MambaBlock`` (:77-192), ``ResidualMambaBlock`` (:195-205),
``BidirectionalMambaBlock`` (:208-237) and ``MultiDirectionalMambaBlock``
(:341-566), with the same constructor arguments, parameter names and
forward semantics, and with ``scan_mode`` passed down to every inner block
(the reference built the inner blocks with the default mode, :202, :223-224,
:403).

Direction blocks do not build permuted copies.  All K directions run as one
batch: one in_proj GEMM (E -> K*2*D_inner), a causal depthwise conv and the
selective scan that read and write through per-direction index tables, the
per-token projections batched over K, and one out_proj GEMM over the
concatenated K*D_inner features, which is also the (atomic-free) sum over
directions (:562-566).
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import directions as _dirs
from .conv import causal_conv_silu
from .scan import get_scan_fn, mode_chunk_len, selective_scan_directions


def _dt_bias_init(d_inner: int, dt_min: float = 1e-3, dt_max: float = 1e-1) -> torch.Tensor:
    """dt_proj bias with softplus(bias) log-uniform in [dt_min, dt_max]."""
    dt = torch.exp(torch.rand(d_inner) * (math.log(dt_max) - math.log(dt_min)) + math.log(dt_min))
    return dt + torch.log(-torch.expm1(-dt))


class MambaBlock(nn.Module):
    """in_proj -> causal depthwise conv1d -> SiLU -> selective scan -> gate ->
    out_proj (mamba_block.py:77-192).  Input / output (B, L, d_model).

    scan_mode: "sequential", "chunked", "parallel", "metal", "metal_train",
    "metal_fused" (the reference's names, mamba_block.py:104-120) or "hip";
    every mode runs the HIP scan.  Unknown names raise ValueError.
    """

    def __init__(self, d_model: int = 384, d_state: int = 16, d_conv: int = 4,
                 expand_factor: int = 2, scan_mode: str = "sequential"):
        super().__init__()
        self.d_model = d_model
        self.d_state = d_state
        self.d_inner = d_model * expand_factor
        self.d_conv = d_conv
        self.scan_mode = scan_mode
        self._scan_fn = get_scan_fn(scan_mode)
        self.dt_rank = math.ceil(d_model / 16)                                 # :136
        self.in_proj = nn.Linear(d_model, 2 * self.d_inner, bias=False)        # :125
        self.conv1d = nn.Conv1d(self.d_inner, self.d_inner, kernel_size=d_conv,
                                padding=d_conv - 1, groups=self.d_inner)        # :129-132
        self.x_proj = nn.Linear(self.d_inner, self.dt_rank + 2 * d_state, bias=False)  # :137
        self.dt_proj = nn.Linear(self.dt_rank, self.d_inner, bias=True)        # :140
        with torch.no_grad():
            self.dt_proj.bias.copy_(_dt_bias_init(self.d_inner))
        A = torch.arange(1, d_state + 1, dtype=torch.float32).repeat(self.d_inner, 1)
        self.A_log = nn.Parameter(torch.log(A))                                # :143-147
        self.D = nn.Parameter(torch.ones(self.d_inner))                        # :150
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=False)           # :153

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _directional_forward([self], x, None, self.scan_mode)


class ResidualMambaBlock(nn.Module):
    """Pre-norm MambaBlock with a residual (mamba_block.py:195-205)."""

    def __init__(self, d_model: int = 384, d_state: int = 16, d_conv: int = 4,
                 expand_factor: int = 2, scan_mode: str = "sequential"):
        super().__init__()
        self.norm = nn.LayerNorm(d_model)
        self.mamba = MambaBlock(d_model, d_state, d_conv, expand_factor, scan_mode)

    def forward(self, x):
        return x + self.mamba(self.norm(x))


class BidirectionalMambaBlock(nn.Module):
    """Forward + reversed-sequence MambaBlocks, summed with a residual
    (mamba_block.py:208-237)."""

    def __init__(self, d_model: int = 384, d_state: int = 16, d_conv: int = 4,
                 expand_factor: int = 2, scan_mode: str = "sequential"):
        super().__init__()
        self.norm = nn.LayerNorm(d_model)
        self.forward_mamba = MambaBlock(d_model, d_state, d_conv, expand_factor, scan_mode)
        self.backward_mamba = MambaBlock(d_model, d_state, d_conv, expand_factor, scan_mode)
        self.scan_mode = scan_mode
        self._tables = {}

    def forward(self, x):
        h = self.norm(x)
        tok = _cached_table(self._tables, 2, x.shape[1], None, x.device)
        return x + _directional_forward([self.forward_mamba, self.backward_mamba], h, tok,
                                        self.scan_mode)


class MultiDirectionalMambaBlock(nn.Module):
    """K independent MambaBlocks, one per scan order, summed with a residual
    (mamba_block.py:341-566).  K = 2, 4 (2D grid), 6 (3D) or 8 (4D).

    When the token count differs from the grid size (a subset of patches),
    the block falls back to forward + backward scans with blocks 0 and 1
    (mamba_block.py:554-559).
    """

    def __init__(self, d_model: int = 384, d_state: int = 16, d_conv: int = 4,
                 expand_factor: int = 2, num_directions: int = 2,
                 grid_shape: Optional[Sequence[int]] = None, scan_mode: str = "sequential"):
        super().__init__()
        if num_directions not in (2, 4, 6, 8):
            raise ValueError(f"num_directions must be 2, 4, 6, or 8, got {num_directions}")
        need = {4: 2, 6: 3, 8: 4}.get(num_directions)
        if need is not None and (grid_shape is None or len(grid_shape) != need):
            raise ValueError(f"K={num_directions} requires a {need}-D grid_shape, got {grid_shape}")
        self.num_directions = num_directions
        self.grid_shape = tuple(grid_shape) if grid_shape is not None else None
        self.scan_mode = scan_mode
        self.norm = nn.LayerNorm(d_model)
        self.mamba_blocks = nn.ModuleList(
            [MambaBlock(d_model, d_state, d_conv, expand_factor, scan_mode)
             for _ in range(num_directions)])
        self._tables = {}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        bsz, n, _ = x.shape
        h = self.norm(x)                                                       # :548
        expected = math.prod(self.grid_shape) if self.grid_shape is not None else n
        if n != expected and self.num_directions > 2:                         # :554-559
            tok = _cached_table(self._tables, 2, n, None, x.device)
            blocks = [self.mamba_blocks[0], self.mamba_blocks[1]]
        else:
            grid = self.grid_shape if self.num_directions > 2 else None
            tok = _cached_table(self._tables, self.num_directions, n, grid, x.device)
            blocks = list(self.mamba_blocks)
        return x + _directional_forward(blocks, h, tok, self.scan_mode)       # :562-566


def _cached_table(cache, K, n, grid, device):
    key = (K, n, grid, str(device))
    if key not in cache:
        cache[key] = _dirs.seq_to_tok_table(K, n, grid).to(device)
    return cache[key]


def _directional_forward(blocks, h, tok, scan_mode):
    """Run len(blocks) MambaBlocks on one (B, N, E) input, block k scanning
    in the order of tok[k], and return the sum of their outputs."""
    K = len(blocks)
    b0 = blocks[0]
    bsz, n, _ = h.shape
    din, ns, R = b0.d_inner, b0.d_state, b0.dt_rank
    W_in = torch.cat([blk.in_proj.weight for blk in blocks], 0) if K > 1 else b0.in_proj.weight
    xz = F.linear(h, W_in).view(bsz, n, K, 2 * din)                            # :165
    xb, z = xz[..., :din], xz[..., din:]                                       # :166-167
    conv_w = torch.cat([blk.conv1d.weight for blk in blocks], 0).view(K, din, b0.d_conv)
    conv_b = torch.cat([blk.conv1d.bias for blk in blocks], 0).view(K, din)
    xc = causal_conv_silu(xb, conv_w, conv_b, tok)                             # :170-171
    W_x = torch.stack([blk.x_proj.weight for blk in blocks], 0)                # (K, R+2N, Din)
    dbc = torch.matmul(xc.permute(2, 0, 1, 3).reshape(K, bsz * n, din),
                       W_x.transpose(1, 2).contiguous())                       # :174
    dbc = dbc.reshape(K, bsz, n, R + 2 * ns).permute(1, 2, 0, 3).contiguous()  # (B, N, K, R+2N)
    dt = dbc[..., :R]                                                          # :175
    Bm = dbc[..., R:R + ns]                                                    # :176
    Cm = dbc[..., R + ns:]                                                     # :177
    W_dt = torch.stack([blk.dt_proj.weight for blk in blocks], 0)              # (K, Din, R)
    b_dt = torch.stack([blk.dt_proj.bias for blk in blocks], 0)                # (K, Din)
    delta = torch.matmul(dt.permute(2, 0, 1, 3).reshape(K, bsz * n, R),
                         W_dt.transpose(1, 2).contiguous())                    # :180
    delta = delta.reshape(K, bsz, n, din).permute(1, 2, 0, 3) + b_dt
    delta = F.softplus(delta).contiguous()                                     # :181
    A = -torch.exp(torch.stack([blk.A_log for blk in blocks], 0))              # :184
    Dv = torch.stack([blk.D for blk in blocks], 0)
    y = selective_scan_directions(xc.contiguous(), delta, A, Bm, Cm, Dv, tok,
                                  chunk_len=mode_chunk_len(scan_mode),
                                  forward_only=(scan_mode == "metal"))         # :187
    y = y * F.silu(z)                                                          # :190
    W_out = torch.cat([blk.out_proj.weight for blk in blocks], 1) if K > 1 else b0.out_proj.weight
    return F.linear(y.reshape(bsz, n, K * din), W_out)                         # :191, :562-566
