"""GPU parity of the remapped causal depthwise conv1d + SiLU against the
reference's formulation in float64 on the CPU: materialised permutation /
reverse of the token sequence (mamba_block.py:254-338, :443-533), torch
conv1d with padding d_conv-1 keeping the first L outputs (:129-132, :170),
SiLU (:171), inverse permutation; gradients by autograd.

Tolerance: |got - ref| <= 1e-5 + 1e-4 * |ref| elementwise for y, dx, dw,
dbias.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import scan_oracle as so
from oracle import torch_ref

pytestmark = pytest.mark.gpu


def _ref(x, w, b, K, grid, kc):
    """x (B, N, K, D) float64 leaf; w (K, D, kc); b (K, D)."""
    bsz, n, _, din = x.shape
    outs = []
    for k in range(K):
        axes, rev = so.direction_axis_order(K, k) if K > 1 else (None, False)
        seq = x[:, :, k, :]
        if axes is not None:
            seq = torch_ref._permute(seq, grid, axes)
        if rev:
            seq = seq.flip(1)
        pre = F.conv1d(seq.transpose(1, 2), w[k].unsqueeze(1), b[k], padding=kc - 1,
                       groups=din)[..., :n].transpose(1, 2)
        out = pre * torch.sigmoid(pre)
        if rev:
            out = out.flip(1)
        if axes is not None:
            out = torch_ref._unpermute(out, grid, axes)
        outs.append(out)
    return torch.stack(outs, dim=2)


def _close(got, ref, name):
    got = got.detach().double().cpu()
    err = (got - ref).abs()
    bound = 1e-5 + 1e-4 * ref.abs()
    assert (err <= bound).all(), f"{name}: max err {float(err.max()):.3e}"


@pytest.mark.parametrize("K,grid,kc", [(1, None, 4), (2, None, 4), (4, (14, 14), 4),
                                       (6, (4, 3, 5), 3), (8, (2, 3, 2, 4), 2), (4, (5, 7), 8)])
def test_conv_parity(cuda, K, grid, kc):
    from mlx_vision_mamba_amd import directions as dirs
    from mlx_vision_mamba_amd.conv import causal_conv_silu
    print(f"case: conv K={K} grid={grid} kc={kc}", flush=True)
    n = int(np.prod(grid)) if grid else 37
    bsz, din = 2, 80
    gen = torch.Generator().manual_seed(K * 10 + kc)
    big = torch.randn(bsz, n, K, 2 * din, generator=gen)   # x is a strided column slice
    w = torch.randn(K, din, kc, generator=gen) * 0.5
    b = torch.randn(K, din, generator=gen) * 0.1
    gy = torch.randn(bsz, n, K, din, generator=gen)
    tok = dirs.seq_to_tok_table(K, n, grid).to(cuda) if K > 1 else None
    bg = big.to(cuda).requires_grad_(True)
    wg = w.to(cuda).requires_grad_(True)
    bbg = b.to(cuda).requires_grad_(True)
    y = causal_conv_silu(bg[..., :din], wg, bbg, tok)
    dbig, dw, db = torch.autograd.grad(y, (bg, wg, bbg), gy.to(cuda))
    xr = big[..., :din].double().clone().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    br = b.double().requires_grad_(True)
    yr = _ref(xr, wr, br, K, grid, kc)
    dxr, dwr, dbr = torch.autograd.grad(yr, (xr, wr, br), gy.double())
    _close(y, yr.detach(), "y")
    _close(dbig[..., :din], dxr, "dx")
    assert not dbig[..., din:].any()
    _close(dw, dwr, "dw")
    _close(db, dbr, "dbias")


@pytest.mark.parametrize("K,n,kc", [(1, 1, 4), (2, 1, 8), (1, 2, 8), (2, 3, 4), (2, 5, 8), (1, 17, 3)])
def test_conv_short_sequences(cuda, K, n, kc):
    """Sequences shorter than the kernel width and than one wave's 16
    positions: every window reaches before position 0 and past the end, so
    the clamped token-row loads and the masks carry the result."""
    from mlx_vision_mamba_amd import directions as dirs
    from mlx_vision_mamba_amd.conv import causal_conv_silu
    print(f"case: conv short K={K} n={n} kc={kc}", flush=True)
    bsz, din = 3, 70
    gen = torch.Generator().manual_seed(n * 10 + kc)
    x = torch.randn(bsz, n, K, din, generator=gen)
    w = torch.randn(K, din, kc, generator=gen) * 0.5
    b = torch.randn(K, din, generator=gen) * 0.1
    gy = torch.randn(bsz, n, K, din, generator=gen)
    tok = dirs.seq_to_tok_table(K, n, None).to(cuda) if K > 1 else None
    xg = x.to(cuda).requires_grad_(True)
    wg = w.to(cuda).requires_grad_(True)
    bg = b.to(cuda).requires_grad_(True)
    y = causal_conv_silu(xg, wg, bg, tok)
    dx, dw, db = torch.autograd.grad(y, (xg, wg, bg), gy.to(cuda))
    xr = x.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    br = b.double().requires_grad_(True)
    yr = _ref(xr, wr, br, K, None, kc)
    dxr, dwr, dbr = torch.autograd.grad(yr, (xr, wr, br), gy.double())
    _close(y, yr.detach(), "y")
    _close(dx, dxr, "dx")
    _close(dw, dwr, "dw")
    _close(db, dbr, "dbias")
