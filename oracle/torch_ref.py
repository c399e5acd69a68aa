"""Torch CPU restatements of the reference -- TEST INFRASTRUCTURE ONLY.

See oracle/__init__.py: only tests/, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py`` use this module.

Two uses:

1. The CPU baseline.  ``scan_sequential`` and ``scan_chunked`` restate the
   reference's ``sequential`` and ``chunked`` scan modes op for op
   (materialised (B,L,D,N) discretisation, a Python loop over time, stack,
   skip term).  Their gradients come from torch autograd, as the reference's
   come from MLX autograd.  ``mlx`` is not installed, so these stand in for
   the reference's CPU run.

2. Module parity.  ``mamba_block``, ``direction_block`` and ``vision_mamba``
   are functional float64 restatements of mamba_block.py:155-192,
   :536-566 and vision_mamba.py:194-224.  They take the parameters of the
   product's modules by name and apply the reference's materialised
   permutations (reshape / transpose / flip), so that the product's
   index-remapped path is checked against the reference's formulation.
   They are pinned by closed forms in tests/test_oracle_blocks.py.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import ref_lib


# ---------------------------------------------------------------------------
# Scan modes
# ---------------------------------------------------------------------------

def scan_sequential(x, delta, A, B, C, D):
    """mamba_block.py:20-74 (the ``sequential`` mode)."""
    bsz, L, d = x.shape
    n = A.shape[1]
    delta_e = delta.unsqueeze(-1)                       # :51
    deltaA = torch.exp(delta_e * A[None, None])         # :52-53
    deltaBx = delta_e * B.unsqueeze(2) * x.unsqueeze(-1)  # :57-59
    h = x.new_zeros((bsz, d, n))                        # :62
    # per-step views taken with one unbind: the same arithmetic as indexing
    # [:, t], without autograd scattering every step's gradient into a
    # full-size zero tensor
    dA_t, dBx_t, C_t = deltaA.unbind(1), deltaBx.unbind(1), C.unbind(1)
    ys = []
    for t in range(L):                                  # :64
        h = dA_t[t] * h + dBx_t[t]                      # :65
        ys.append((h * C_t[t].unsqueeze(1)).sum(-1))    # :67
    y = torch.stack(ys, dim=1)                          # :70
    return y + x * D                                    # :73


def scan_chunked(x, delta, A, B, C, D, chunk_size=32):
    """mamba_fast.py:17-75 (the ``chunked`` mode)."""
    bsz, L, d = x.shape
    n = A.shape[1]
    delta_e = delta.unsqueeze(-1)
    deltaA = torch.exp(delta_e * A[None, None])          # :41-43
    deltaBx = delta_e * B.unsqueeze(2) * x.unsqueeze(-1)  # :45-47
    h = x.new_zeros((bsz, d, n))                          # :50
    parts = []
    for c0 in range(0, L, chunk_size):                    # :53
        c1 = min(c0 + chunk_size, L)
        dA_c = deltaA[:, c0:c1].unbind(1)
        dBx_c = deltaBx[:, c0:c1].unbind(1)
        C_c = C[:, c0:c1].unbind(1)
        ys = []
        for t in range(c1 - c0):                          # :64
            h = dA_c[t] * h + dBx_c[t]
            ys.append((h * C_c[t].unsqueeze(1)).sum(-1))
        parts.append(torch.stack(ys, dim=1))              # :70
    return torch.cat(parts, dim=1) + x * D                # :73-74


class _OracleScanFn(torch.autograd.Function):
    """The float64 C oracle (scan_ref.c, float64-input forms) as a torch op:
    forward mamba_block.py:45-74, VJP mamba_metal_fused.py:66-145,
    213-224.  Same function and gradients as ``scan_sequential`` (checked
    in tests/test_oracle_blocks.py), without a Python step per position, so
    the module restatements run at full sequence lengths in seconds."""

    @staticmethod
    def forward(ctx, x, delta, A, B, C, D):
        ctx.save_for_backward(x, delta, A, B, C, D)
        arrs = [t.detach().numpy() for t in (x, delta, A, B, C, D)]
        return torch.from_numpy(ref_lib.scan_fwd_f64(*arrs))

    @staticmethod
    def backward(ctx, gy):
        arrs = [t.detach().numpy() for t in ctx.saved_tensors]
        grads = ref_lib.scan_vjp_f64(*arrs, gy.detach().double().numpy())
        return tuple(torch.from_numpy(g) for g in grads)


def scan_oracle_c(x, delta, A, B, C, D):
    """float64 CPU scan with autograd through the C oracle; a drop-in for
    ``scan_sequential`` in the module restatements (float64 tensors)."""
    for t in (x, delta, A, B, C, D):
        if t.dtype != torch.float64 or t.device.type != "cpu":
            raise ValueError("scan_oracle_c takes float64 CPU tensors")
    return _OracleScanFn.apply(x, delta, A, B, C, D)


# ---------------------------------------------------------------------------
# Module restatements (float64 by default)
# ---------------------------------------------------------------------------

def _p(params, name, dtype):
    return params[name].detach().to(dtype).requires_grad_(params[name].requires_grad)


def mamba_block(params, prefix, x, d_state, d_conv, scan=scan_sequential):
    """MambaBlock.__call__, mamba_block.py:155-192, on a (B,L,E) sequence.

    ``params`` maps the product module's parameter names to tensors (already
    float64 leaves); ``prefix`` selects one block.
    """
    W_in = params[prefix + "in_proj.weight"]
    conv_w = params[prefix + "conv1d.weight"]     # (Din, 1, d_conv)
    conv_b = params[prefix + "conv1d.bias"]
    W_x = params[prefix + "x_proj.weight"]
    W_dt = params[prefix + "dt_proj.weight"]
    b_dt = params[prefix + "dt_proj.bias"]
    A_log = params[prefix + "A_log"]
    Dp = params[prefix + "D"]
    W_out = params[prefix + "out_proj.weight"]
    bsz, L, _ = x.shape
    d_inner = W_out.shape[1]
    dt_rank = W_dt.shape[1]
    xz = x @ W_in.T                                            # :165
    xb, z = xz[..., :d_inner], xz[..., d_inner:]               # :166-167
    # MLX Conv1d with padding d_conv-1 on both sides, then keep the first L
    # outputs (:129-132, :170): output t sees inputs t-d_conv+1 .. t, tap j
    # weighting input t - (d_conv - 1) + j (a cross-correlation), written
    # as a sum over the taps of the zero-padded sequence
    xp = F.pad(xb, (0, 0, d_conv - 1, 0))
    w = conv_w[:, 0, :]
    xc = conv_b + sum(xp[:, j:j + L] * w[:, j] for j in range(d_conv))
    xc = xc * torch.sigmoid(xc)                                # :171 SiLU
    dbc = xc @ W_x.T                                           # :174
    dt = dbc[..., :dt_rank]                                    # :175
    Bm = dbc[..., dt_rank:dt_rank + d_state]                   # :176
    Cm = dbc[..., dt_rank + d_state:]                          # :177
    delta = dt @ W_dt.T + b_dt                                 # :180
    delta = torch.log(1.0 + torch.exp(delta))                  # :181 softplus
    A = -torch.exp(A_log)                                      # :184
    y = scan(xc, delta, A, Bm, Cm, Dp)                         # :187
    y = y * (z * torch.sigmoid(z))                             # :190
    return y @ W_out.T                                         # :191


def layer_norm(params, prefix, x, eps=1e-5):
    """nn.LayerNorm with affine weight and bias (MLX default eps 1e-5)."""
    return F.layer_norm(x, (x.shape[-1],), params[prefix + "weight"],
                        params[prefix + "bias"], eps)


def _permute(h, grid_shape, axes_order):
    """_permute_2d_col_major / _permute_3d_axis / _permute_4d_axis,
    mamba_block.py:254-264, :277-290, :311-323."""
    bsz, n, e = h.shape
    nd = len(grid_shape)
    h = h.reshape(bsz, *grid_shape, e)
    perm = (0,) + tuple(a + 1 for a in axes_order) + (nd + 1,)
    return h.permute(perm).reshape(bsz, n, e)


def _unpermute(h, grid_shape, axes_order):
    """The matching inverses, mamba_block.py:267-274, :293-308, :326-338."""
    bsz, n, e = h.shape
    nd = len(grid_shape)
    permuted = tuple(grid_shape[a] for a in axes_order)
    h = h.reshape(bsz, *permuted, e)
    inv = [0] * nd
    for i, a in enumerate(axes_order):
        inv[a] = i
    perm = (0,) + tuple(a + 1 for a in inv) + (nd + 1,)
    return h.permute(perm).reshape(bsz, n, e)


_AXES = {
    2: [None],
    4: [None, (1, 0)],
    6: [None, (1, 0, 2), (2, 0, 1)],
    8: [None, (1, 0, 2, 3), (2, 0, 1, 3), (3, 0, 1, 2)],
}


def direction_block(params, prefix, x, num_directions, grid_shape, d_state,
                    d_conv, scan=scan_sequential):
    """MultiDirectionalMambaBlock.__call__ / _apply_direction,
    mamba_block.py:407-566 (materialised permutations and reverses)."""
    bsz, n, _ = x.shape
    h = layer_norm(params, prefix + "norm.", x)                # :548
    expected = 1
    for gdim in (grid_shape or (n,)):
        expected *= gdim
    K = num_directions
    if n != expected and K > 2:                                # :554-559
        y_f = mamba_block(params, prefix + "mamba_blocks.0.", h, d_state, d_conv, scan)
        y_b = mamba_block(params, prefix + "mamba_blocks.1.", h.flip(1), d_state, d_conv, scan).flip(1)
        return x + y_f + y_b
    y = None
    for k in range(K):                                         # :562-564
        pair, rev = divmod(k, 2)
        axes = _AXES[K][pair]
        seq = h if axes is None else _permute(h, grid_shape, axes)
        if rev:
            seq = seq.flip(1)
        out = mamba_block(params, f"{prefix}mamba_blocks.{k}.", seq, d_state, d_conv, scan)
        if rev:
            out = out.flip(1)
        if axes is not None:
            out = _unpermute(out, grid_shape, axes)
        y = out if y is None else y + out
    return x + y                                               # :566


def bidirectional_block(params, prefix, x, d_state, d_conv, scan=scan_sequential):
    """BidirectionalMambaBlock.__call__, mamba_block.py:226-237."""
    h = layer_norm(params, prefix + "norm.", x)
    y_f = mamba_block(params, prefix + "forward_mamba.", h, d_state, d_conv, scan)
    y_b = mamba_block(params, prefix + "backward_mamba.", h.flip(1), d_state, d_conv, scan).flip(1)
    return x + y_f + y_b


def vision_mamba(params, x, *, input_dim, patch_size, depth, grid_shape,
                 d_state, d_conv, temporal_patch_size=1, scan=scan_sequential,
                 patch_indices=None):
    """VisionMamba.__call__, vision_mamba.py:194-224, with PatchEmbed
    (vit.py:62-67), PatchEmbed3D (vit.py:87-92) and PatchEmbed4D
    (vision_mamba.py:65-94), all channel-last."""
    if x.ndim != 3:
        w = params["patch_embed.proj.weight"]
        b = params["patch_embed.proj.bias"]
        if input_dim == 2:
            out = F.conv2d(x.permute(0, 3, 1, 2), w, b, stride=patch_size)
            x = out.flatten(2).transpose(1, 2)
        elif input_dim == 3:
            out = F.conv3d(x.permute(0, 4, 1, 2, 3), w, b, stride=patch_size)
            x = out.flatten(2).transpose(1, 2)
        else:
            bsz, T, Dd, H, W, C = x.shape
            tp = temporal_patch_size
            if tp > 1:
                x = x.reshape(bsz, T // tp, tp, Dd, H, W, C).permute(0, 1, 3, 4, 5, 2, 6)
                x = x.reshape(bsz, T // tp, Dd, H, W, tp * C)
            t_out = T // tp
            x = x.reshape(bsz * t_out, Dd, H, W, -1)
            out = F.conv3d(x.permute(0, 4, 1, 2, 3), w, b, stride=patch_size)
            E = out.shape[1]
            out = out.permute(0, 2, 3, 4, 1)                    # channel-last
            x = out.reshape(bsz, -1, E)
    pos = params["pos_embed"]
    x = x + (pos[:, patch_indices, :] if patch_indices is not None else pos)
    K = {2: 4, 3: 6, 4: 8}[input_dim]
    for i in range(depth):
        x = direction_block(params, f"blocks.{i}.", x, K, grid_shape, d_state, d_conv, scan)
    return layer_norm(params, "norm.", x)


def params_from_module(module, dtype=torch.float64):
    """Detached float64 copies of a module's parameters, as grad leaves."""
    return {k: v.detach().to("cpu", dtype).clone().requires_grad_(True)
            for k, v in module.named_parameters()}


def softplus_inverse(dt):
    """dt_bias such that softplus(dt_bias) == dt."""
    return dt + torch.log(-torch.expm1(-dt))


def dt_rank_for(d_model):
    """mamba_block.py:136."""
    return math.ceil(d_model / 16)
