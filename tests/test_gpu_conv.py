"""GPU parity of the remapped causal depthwise conv1d + SiLU against the
reference's formulation in float64 on the CPU: materialised permutation /
reverse of the token sequence (mamba_block.py:254-338, :443-533), torch
conv1d with padding d_conv-1 keeping the first L outputs (:129-132, :170),
SiLU (:171), inverse permutation; gradients by autograd.

Tolerance: |got - ref| <= 1e-5 + 1e-4 * |ref| elementwise for y, dx, dw,
dbias.  At the VisionMamba-2D step shape (batch 32, K=4 on 14x14 tokens,
768 channels) dw and dbias are 6272-row float32 sums, and the bound adds
32 * 2^-24 * S per element, S being the error magnitude of the element from
the oracle's running error analysis (the TC ops of oracle/torch_ref.py):
the magnitudes of the terms that form it, each with the errors of its
factors (for dx, dw and dbias the error of silu'(pre) from that of pre
included).
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


def _ref_tc(x, w, b, K, grid, kc):
    """_ref on (value, error magnitude) pairs (oracle/torch_ref.py TC ops):
    x (B, N, K, D), w (K, D, kc), b (K, D) as TC pairs."""
    n = x.v.shape[1]
    outs = []
    for k in range(K):
        axes, rev = so.direction_axis_order(K, k) if K > 1 else (None, False)
        seq = x[:, :, k, :]
        if axes is not None:
            seq = seq.map(lambda t: torch_ref._permute(t, grid, axes))
        if rev:
            seq = seq.flip(1)
        xp = seq.map(lambda t: F.pad(t, (0, 0, kc - 1, 0)))
        pre = b[k]
        for j in range(kc):
            pre = pre + torch_ref.tc_mul(xp[:, j:j + n], w[k][:, j])
        out = torch_ref.tc_pointwise("silu", pre)
        if rev:
            out = out.flip(1)
        if axes is not None:
            out = out.map(lambda t: torch_ref._unpermute(t, grid, axes))
        outs.append(out)
    return torch_ref.TC(torch.stack([o.v for o in outs], 2), torch.stack([o.m for o in outs], 2))


def _close(got, ref, name, S=None):
    got = got.detach().double().cpu()
    err = (got - ref).abs()
    bound = 1e-5 + 1e-4 * ref.abs()
    if S is not None:
        bound = bound + 32 * 2.0 ** -24 * S
        print(f"{name}: worst err / (2^-24 S) = {float((err / (2.0 ** -24 * S)).max()):.3f}")
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


def test_conv_parity_at_the_step_shape(cuda):
    """The VisionMamba-2D layer's conv: batch 32, K=4 directions on the
    14x14 token grid, 768 channels, width 4, x a column slice of the in_proj
    output (B, N, K, 2D) as in the block; dw and dbias sum 6272 rows."""
    from mlx_vision_mamba_amd import directions as dirs
    from mlx_vision_mamba_amd.conv import causal_conv_silu
    print("case: conv at the step shape B=32 K=4 14x14 D=768", flush=True)
    bsz, K, grid, kc, din = 32, 4, (14, 14), 4, 768
    n = 196
    gen = torch.Generator().manual_seed(77)
    big = torch.randn(bsz, n, K, 2 * din, generator=gen)
    w = torch.randn(K, din, kc, generator=gen) * 0.5
    b = torch.randn(K, din, generator=gen) * 0.1
    gy = torch.randn(bsz, n, K, din, generator=gen)
    tok = dirs.seq_to_tok_table(K, n, grid).to(cuda)
    bg = big.to(cuda).requires_grad_(True)
    wg = w.to(cuda).requires_grad_(True)
    bbg = b.to(cuda).requires_grad_(True)
    y = causal_conv_silu(bg[..., :din], wg, bbg, tok)
    dbig, dw, db = torch.autograd.grad(y, (bg, wg, bbg), gy.to(cuda))
    x = big[..., :din].double()
    xr, wr, br = x.clone().requires_grad_(True), w.double().requires_grad_(True), b.double().requires_grad_(True)
    yr = _ref(xr, wr, br, K, grid, kc)
    dxr, dwr, dbr = torch.autograd.grad(yr, (xr, wr, br), gy.double())
    TC = torch_ref.TC
    leaves = [t.detach().clone().requires_grad_(True) for t in (x, wr, br)]
    mags = [t.detach().abs().requires_grad_(True) for t in (x, wr, br)]
    out = _ref_tc(*[TC(v, m) for v, m in zip(leaves, mags)], K, grid, kc)
    ((gy.double() * out.v).sum() + (gy.double().abs() * out.m).sum()).backward()
    My = out.m.detach()
    Mx, aw, ab = mags
    _close(y, yr.detach(), "y", My.detach())
    _close(dbig[..., :din], dxr, "dx", Mx.grad)
    assert not dbig[..., din:].any()
    _close(dw, dwr, "dw", aw.grad)
    _close(db, dbr, "dbias", ab.grad)
