"""Pins the module restatements of the oracle (oracle/torch_ref.py:
``mamba_block``, ``layer_norm``, ``direction_block``, ``bidirectional_block``
and ``vision_mamba``) by closed forms built from other routines.

With A_log = -30 every decay exp(delta * A) equals 1 to float64 precision
(A = -9.4e-14), so the selective scan reduces to a prefix sum
(``np.cumsum``) and the whole block has a closed form:
  * the causal depthwise conv is ``np.convolve`` with the reversed taps
    (MLX Conv1d is a cross-correlation padded by d_conv-1 on both sides and
    cut to the first L outputs, mamba_block.py:129-132, :170);
  * the scan output is y_t = C_t . cumsum_s<=t(delta_s B_s x_s) + D x_t;
  * the direction orders are numpy reshape / transpose / ravel of
    ``np.arange`` (mamba_block.py:244-338, :407-533), applied as a gather
    and undone as a scatter.
At two tokens the decay is kept (A_log ~ 0) and the scan is written out by
hand, which pins A = -exp(A_log) as well.  Each closed form is also shown
to be sensitive to the plausible mistakes (B <-> C slices swapped, conv
taps reversed, the dt | B | C split shifted by one column, LayerNorm weight
and bias swapped, a direction's order not undone): the mutated closed form
differs from the restatement by far more than the tolerance.
"""

import math

import numpy as np
import pytest
import torch

from mlx_vision_mamba_amd import mamba_block as mb
from mlx_vision_mamba_amd import vision_mamba as vm
from oracle import torch_ref

RTOL, ATOL = 1e-10, 1e-12


def _silu(v):
    return v / (1.0 + np.exp(-v))


def _softplus(v):
    return np.logaddexp(0.0, v)


def _np(t):
    return t.detach().double().numpy()


def _ln(x, w, b, eps=1e-5):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def _params(module, seed, a_log=-30.0):
    """float64 leaves of a product module's parameters with randomised
    LayerNorm affines and conv taps, and A_log set to ``a_log``."""
    gen = torch.Generator().manual_seed(seed)
    p = torch_ref.params_from_module(module)
    for k in list(p):
        if k.endswith("A_log"):
            p[k] = torch.full_like(p[k], a_log).requires_grad_(True)
        elif k.endswith("norm.weight") or k.endswith("norm.bias") or k.endswith("conv1d.bias") \
                or k.endswith(".D"):
            p[k] = (torch.randn(p[k].shape, generator=gen, dtype=torch.float64) * 0.5
                    + (1.0 if k.endswith("weight") or k.endswith(".D") else 0.0)).requires_grad_(True)
        elif k.endswith("conv1d.weight"):
            p[k] = torch.randn(p[k].shape, generator=gen, dtype=torch.float64).requires_grad_(True)
    return p


def _block_np(p, pre, x, *, swap_bc=False, flip_taps=False, split_shift=0, decay_one=True):
    """Closed form of MambaBlock.__call__ (mamba_block.py:155-192) with every
    decay equal to 1: np.convolve for the conv, np.cumsum for the scan."""
    g = {k[len(pre):]: _np(v) for k, v in p.items() if k.startswith(pre)}
    W_in, conv_w, conv_b = g["in_proj.weight"], g["conv1d.weight"], g["conv1d.bias"]
    W_x, W_dt, b_dt, Dp = g["x_proj.weight"], g["dt_proj.weight"], g["dt_proj.bias"], g["D"]
    W_out = g["out_proj.weight"]
    bsz, L, _ = x.shape
    din, R, N = W_out.shape[1], W_dt.shape[1], g["A_log"].shape[1]
    xz = x @ W_in.T
    xb, z = xz[..., :din], xz[..., din:]
    taps = conv_w[:, 0, :]
    if flip_taps:
        taps = taps[:, ::-1]
    xc = np.empty_like(xb)
    for b in range(bsz):
        for d in range(din):
            xc[b, :, d] = np.convolve(xb[b, :, d], taps[d, ::-1])[:L]
    xc = _silu(xc + conv_b)
    dbc = xc @ W_x.T
    s = R + split_shift
    dt, Bm, Cm = dbc[..., :R], dbc[..., s:s + N], dbc[..., s + N:s + 2 * N]
    if swap_bc:
        Bm, Cm = Cm, Bm
    delta = _softplus(dt @ W_dt.T + b_dt)
    if decay_one:
        h = np.cumsum(delta[..., None] * Bm[:, :, None, :] * xc[..., None], axis=1)
        y = np.einsum("bldn,bln->bld", h, Cm) + Dp * xc
    else:
        # two tokens, decay kept: h_0 = d0 B0 x0; h_1 = exp(d1 A) h_0 + d1 B1 x1
        assert L == 2
        A = -np.exp(g["A_log"])                                  # (din, N)
        h0 = delta[:, 0, :, None] * Bm[:, 0, None, :] * xc[:, 0, :, None]
        h1 = np.exp(delta[:, 1, :, None] * A) * h0 + \
            delta[:, 1, :, None] * Bm[:, 1, None, :] * xc[:, 1, :, None]
        y = np.stack([(h0 * Cm[:, 0, None, :]).sum(-1), (h1 * Cm[:, 1, None, :]).sum(-1)], 1)
        y = y + Dp * xc
    y = y * _silu(z)
    return y @ W_out.T


def _orders(K, grid, n):
    """Scan order (token index at each scan position) of every direction,
    from numpy reshape / transpose / ravel (mamba_block.py:407-533)."""
    axes = {2: [None], 4: [None, (1, 0)], 6: [None, (1, 0, 2), (2, 0, 1)],
            8: [None, (1, 0, 2, 3), (2, 0, 1, 3), (3, 0, 1, 2)]}[K]
    out = []
    for k in range(K):
        a = axes[k // 2]
        o = np.arange(n) if a is None else np.arange(n).reshape(grid).transpose(a).ravel()
        out.append(o[::-1] if k % 2 else o)
    return out


def _direction_np(p, pre, x, K, grid, *, unscatter=True, ln_swap=False):
    """Closed form of MultiDirectionalMambaBlock.__call__ (mamba_block.py:536-566):
    x + sum_k scatter_k(block_k(gather_k(LayerNorm(x))))."""
    w, b = _np(p[pre + "norm.weight"]), _np(p[pre + "norm.bias"])
    h = _ln(x, b, w) if ln_swap else _ln(x, w, b)
    n = x.shape[1]
    if grid is not None and n != math.prod(grid) and K > 2:
        K, grid = 2, None                                       # :554-559 fallback
    y = np.zeros_like(x)
    for k, order in enumerate(_orders(K, grid, n)):
        out_seq = _block_np(p, f"{pre}mamba_blocks.{k}.", h[:, order])
        if unscatter:
            y[:, order] += out_seq
        else:
            y += out_seq
    return x + y


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def _far(a, b):
    """The mutated closed form must miss the restatement by far more than
    the tolerance."""
    return np.max(np.abs(a - b)) > 1e3 * (ATOL + RTOL * np.max(np.abs(b)))


# --------------------------------------------------------------- MambaBlock

def test_mamba_block_closed_form_decay_one():
    torch.manual_seed(0)
    blk = mb.MambaBlock(d_model=6, d_state=4, d_conv=4)
    p = _params(blk, seed=1)
    for k in ("in_proj.weight", "x_proj.weight"):
        p[k] = (p[k] * 3.0).detach().requires_grad_(True)       # O(1) scan inputs
    x = _rand((2, 7, 6), 2)
    got = _np(torch_ref.mamba_block(p, "", torch.tensor(x), d_state=4, d_conv=4))
    ref = _block_np(p, "", x)
    np.testing.assert_allclose(got, ref, rtol=RTOL, atol=ATOL)
    for mut in (dict(swap_bc=True), dict(flip_taps=True), dict(split_shift=-1)):
        assert _far(_block_np(p, "", x, **mut), got), mut


def test_mamba_block_two_tokens_with_decay():
    """A = -exp(A_log) with A_log ~ N(1, 0.3): decays far from 1."""
    torch.manual_seed(3)
    blk = mb.MambaBlock(d_model=5, d_state=3, d_conv=3)
    p = _params(blk, seed=4)
    gen = torch.Generator().manual_seed(5)
    p["A_log"] = (torch.randn(p["A_log"].shape, generator=gen, dtype=torch.float64) * 0.3
                  + 1.0).requires_grad_(True)
    p["dt_proj.bias"] = torch.full_like(p["dt_proj.bias"], 0.5).requires_grad_(True)
    x = _rand((3, 2, 5), 6)
    got = _np(torch_ref.mamba_block(p, "", torch.tensor(x), d_state=3, d_conv=3))
    ref = _block_np(p, "", x, decay_one=False)
    np.testing.assert_allclose(got, ref, rtol=RTOL, atol=ATOL)
    # the decay matters here: the decay-1 form is far off
    assert _far(_block_np(p, "", x, decay_one=True), got)
    for mut in (dict(swap_bc=True, decay_one=False), dict(flip_taps=True, decay_one=False)):
        assert _far(_block_np(p, "", x, **mut), got), mut


def test_layer_norm_textbook():
    w, b = _rand(9, 7) * 0.5 + 1.0, _rand(9, 8) * 0.5
    x = _rand((4, 9), 9) * 3.0 + 1.5
    p = {"n.weight": torch.tensor(w), "n.bias": torch.tensor(b)}
    got = _np(torch_ref.layer_norm(p, "n.", torch.tensor(x)))
    np.testing.assert_allclose(got, _ln(x, w, b), rtol=1e-12, atol=1e-12)
    assert _far(_ln(x, b, w), got)


# ---------------------------------------------------------- direction blocks

@pytest.mark.parametrize("K,grid,n", [(4, (2, 3), 6), (6, (2, 3, 2), 12), (8, (2, 2, 1, 3), 12),
                                      (2, None, 5), (6, (2, 3, 2), 7)])
def test_direction_block_closed_form(K, grid, n):
    torch.manual_seed(10 + K)
    blk = mb.MultiDirectionalMambaBlock(d_model=4, d_state=2, d_conv=4, num_directions=K,
                                        grid_shape=grid)
    p = _params(blk, seed=K)
    x = _rand((2, n, 4), 11)
    got = _np(torch_ref.direction_block(p, "", torch.tensor(x), K, grid, d_state=2, d_conv=4))
    ref = _direction_np(p, "", x, K, grid)
    np.testing.assert_allclose(got, ref, rtol=RTOL, atol=ATOL)
    assert _far(_direction_np(p, "", x, K, grid, ln_swap=True), got)
    if K > 2 and n == math.prod(grid):
        assert _far(_direction_np(p, "", x, K, grid, unscatter=False), got)


def test_bidirectional_block_closed_form():
    torch.manual_seed(20)
    blk = mb.BidirectionalMambaBlock(d_model=4, d_state=3, d_conv=4)
    p = _params(blk, seed=21)
    x = _rand((2, 6, 4), 22)
    got = _np(torch_ref.bidirectional_block(p, "", torch.tensor(x), d_state=3, d_conv=4))
    h = _ln(x, _np(p["norm.weight"]), _np(p["norm.bias"]))
    ref = x + _block_np(p, "forward_mamba.", h) + \
        _block_np(p, "backward_mamba.", h[:, ::-1])[:, ::-1]
    np.testing.assert_allclose(got, ref, rtol=RTOL, atol=ATOL)
    assert _far(x + _block_np(p, "forward_mamba.", h) + _block_np(p, "backward_mamba.", h[:, ::-1]),
                got)


# ----------------------------------------------------------------- encoder

def _patch_embed_brute(x, w, b, p, tp, input_dim):
    """Patch embedding by an explicit loop over tokens: token order is
    row-major over the patch grid (and over time groups first in 4D), each
    token the dot product of its patch with the conv weight (vit.py:48-92,
    vision_mamba.py:25-94; in 4D frame f*tp + i of a group feeds weight
    channel i*C + c)."""
    E = w.shape[0]
    if input_dim == 2:
        bsz, H, W, C = x.shape
        x = x.reshape(bsz, 1, 1, H, W, C)
    elif input_dim == 3:
        bsz, Dd, H, W, C = x.shape
        x = x.reshape(bsz, 1, Dd, H, W, C)
    bsz, T, Dd, H, W, C = x.shape
    tg = T // tp
    sp = (1,) if input_dim == 2 else (p,)
    gd, gh, gw = Dd // sp[0], H // p, W // p
    toks = []
    for bb in range(bsz):
        row = []
        for f in range(tg):
            for i in range(gd):
                for j in range(gh):
                    for k in range(gw):
                        acc = b.copy()
                        for e in range(E):
                            s = 0.0
                            for ti in range(tp):
                                for c in range(C):
                                    blk = x[bb, f * tp + ti, i * sp[0]:(i + 1) * sp[0],
                                            j * p:(j + 1) * p, k * p:(k + 1) * p, c]
                                    if input_dim == 2:
                                        wk = w[e, c]                     # (p, p)
                                        s += float(np.sum(blk[0] * wk))
                                    else:
                                        wk = w[e, ti * C + c]            # (p, p, p)
                                        s += float(np.sum(blk * wk))
                            acc[e] += s
                        row.append(acc)
        toks.append(row)
    return np.array(toks)


@pytest.mark.parametrize("input_dim", [2, 3, 4])
def test_vision_mamba_closed_form(input_dim):
    torch.manual_seed(30 + input_dim)
    if input_dim == 2:
        model = vm.VisionMamba(img_size=8, patch_size=4, in_channels=2, embed_dim=4, depth=1,
                               d_state=2, input_dim=2)
        x = _rand((2, 8, 8, 2), 31)
        tp, grid = 1, (2, 2)
    elif input_dim == 3:
        model = vm.VisionMamba(img_size=4, patch_size=2, embed_dim=4, depth=1, d_state=2,
                               input_dim=3)
        x = _rand((1, 4, 4, 4, 1), 32)
        tp, grid = 1, (2, 2, 2)
    else:
        model = vm.VisionMamba(img_size=4, patch_size=2, in_channels=1, embed_dim=4, depth=1,
                               d_state=2, input_dim=4, temporal_patch_size=2,
                               num_temporal_frames=4)
        x = _rand((1, 4, 4, 4, 4, 1), 33)
        tp, grid = 2, (2, 2, 2, 2)
    assert tuple(model.grid_shape) == grid
    p = _params(model, seed=34)
    K = {2: 4, 3: 6, 4: 8}[input_dim]
    got = _np(torch_ref.vision_mamba(p, torch.tensor(x), input_dim=input_dim, patch_size=model.patch_size,
                                     depth=1, grid_shape=grid, d_state=2, d_conv=4,
                                     temporal_patch_size=tp))
    tok = _patch_embed_brute(x, _np(p["patch_embed.proj.weight"]), _np(p["patch_embed.proj.bias"]),
                             model.patch_size, tp, input_dim)
    tok = tok + _np(p["pos_embed"])
    tok = _direction_np(p, "blocks.0.", tok, K, grid)
    ref = _ln(tok, _np(p["norm.weight"]), _np(p["norm.bias"]))
    np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-11)


@pytest.mark.parametrize("K,grid", [(4, (3, 5)), (6, (2, 3, 4))])
def test_c_oracle_scan_op_equals_the_sequential_restatement(K, grid):
    """torch_ref.scan_oracle_c (the float64 C oracle as a torch op, used
    by the full-size module checks) gives the same block output and
    gradients as the op-for-op sequential restatement."""
    torch.manual_seed(40 + K)
    blk = mb.MultiDirectionalMambaBlock(d_model=16, num_directions=K, grid_shape=grid)
    x = torch.randn(2, int(np.prod(grid)), 16, dtype=torch.float64)
    gy = torch.randn(2, int(np.prod(grid)), 16, dtype=torch.float64)
    res = []
    for scan in (torch_ref.scan_sequential, torch_ref.scan_oracle_c):
        p = torch_ref.params_from_module(blk)
        xr = x.clone().requires_grad_(True)
        y = torch_ref.direction_block(p, "", xr, K, grid, 16, 4, scan=scan)
        y.backward(gy)
        res.append([y.detach(), xr.grad] + [p[k].grad for k in sorted(p)])
    for a, b in zip(*res):
        np.testing.assert_allclose(_np(a), _np(b), rtol=1e-10, atol=1e-12)
    with pytest.raises(ValueError):
        torch_ref.scan_oracle_c(*[torch.zeros(1, 2, 3)] * 2, torch.zeros(3, 4),
                                *[torch.zeros(1, 2, 4)] * 2, torch.zeros(3))


# ------------------------------------------------- magnitude companions

from tests import module_bounds as mbd  # noqa: E402


def _mag_case(kind):
    """(module, input shape, restatement, TC restatement) for each kind."""
    if kind == "mamba":
        blk = mb.MambaBlock(d_model=16, d_state=16)
        return blk, (2, 9, 16), (lambda p, x: torch_ref.mamba_block(p, "", x, 16, 4)), \
            (lambda P, X: torch_ref.mamba_block_tc(P, "", X, 16, 4))
    if kind == "residual":
        blk = mb.ResidualMambaBlock(d_model=16)
        return blk, (2, 9, 16), (lambda p, x: x + torch_ref.mamba_block(
            p, "mamba.", torch_ref.layer_norm(p, "norm.", x), 16, 4)), \
            (lambda P, X: torch_ref.residual_block_tc(P, "", X, 16, 4))
    if kind == "bidirectional":
        blk = mb.BidirectionalMambaBlock(d_model=16)
        return blk, (2, 9, 16), (lambda p, x: torch_ref.bidirectional_block(p, "", x, 16, 4)), \
            (lambda P, X: torch_ref.bidirectional_block_tc(P, "", X, 16, 4))
    if kind.startswith("dir"):
        K, grid, n = {"dir2": (2, None, 7), "dir4": (4, (3, 4), 12), "dir6": (6, (2, 3, 2), 12),
                      "dir8": (8, (2, 1, 2, 3), 12), "dir4fallback": (4, (3, 4), 5)}[kind]
        blk = mb.MultiDirectionalMambaBlock(d_model=16, num_directions=K, grid_shape=grid)
        return blk, (2, n, 16), (lambda p, x: torch_ref.direction_block(p, "", x, K, grid, 16, 4)), \
            (lambda P, X: torch_ref.direction_block_tc(P, "", X, K, grid, 16, 4))
    dim = int(kind[-2])
    kw = {2: {}, 3: {}, 4: {"num_temporal_frames": 4, "temporal_patch_size": 2}}[dim]
    shape = {2: (2, 16, 16, 1), 3: (1, 8, 8, 8, 1), 4: (1, 4, 8, 8, 8, 1)}[dim]
    model = vm.VisionMamba(img_size=shape[-2], patch_size=4, embed_dim=16, depth=2, input_dim=dim,
                           **kw)
    common = dict(input_dim=dim, patch_size=4, depth=2, grid_shape=model.grid_shape, d_state=16,
                  d_conv=4, temporal_patch_size=kw.get("temporal_patch_size", 1))
    return model, shape, (lambda p, x: torch_ref.vision_mamba(p, x, **common)), \
        (lambda P, X: torch_ref.vision_mamba_tc(P, X, **common))


MAG_KINDS = ["mamba", "residual", "bidirectional", "dir2", "dir4", "dir6", "dir8", "dir4fallback",
             "vm2d", "vm3d", "vm4d"]


@pytest.mark.parametrize("kind", MAG_KINDS)
def test_error_magnitudes_bound_the_restatements(kind):
    """The ``*_tc`` running error analysis: its value channel reproduces the
    restatement's output and every gradient (its backward formulas are
    checked against torch autograd of the restatement); every magnitude is
    at least the absolute value it stands for; and the restatement
    evaluated in float32 (the reference's precision) is within
    2 * 2^-24 * S of the float64 values, element by element (the module
    parity tests allow 8 * 2^-24 * S, module_bounds.C_MOD)."""
    torch.manual_seed(70)
    module, shape, ref_fn, tc_fn = _mag_case(kind)
    x = torch.randn(*shape, dtype=torch.float64)
    p = torch_ref.params_from_module(module)
    xr = x.clone().requires_grad_(True)
    y = ref_fn(p, xr)
    G = torch.randn(y.shape, dtype=torch.float64)
    y.backward(G)
    val, grads, S = torch_ref.run_tc(tc_fn, torch_ref.params_from_module(module), x, G)
    np.testing.assert_allclose(_np(val), _np(y), rtol=1e-12, atol=1e-13)
    refs = {"output": y.detach(), "input grad": xr.grad}
    refs.update({f"grad {k}": v.grad for k, v in p.items() if v.grad is not None})
    assert set(refs) == set(S)
    for name, r in refs.items():
        if name != "output":
            np.testing.assert_allclose(_np(grads[name]), _np(r), rtol=1e-10, atol=1e-12, err_msg=name)
        assert bool((S[name] >= r.abs() * (1 - 1e-12)).all()), name
    # float32 evaluation of the same restatement
    p32 = {k: v.detach().float().requires_grad_(True) for k, v in p.items()}
    x32 = x.float().requires_grad_(True)
    y32 = ref_fn(p32, x32)
    y32.backward(G.float())
    got = {"output": y32.detach(), "input grad": x32.grad}
    got.update({f"grad {k}": v.grad for k, v in p32.items() if v.grad is not None})
    for name, r in refs.items():
        mbd.check(name, got[name], r, S[name], c=2, cap=False)
