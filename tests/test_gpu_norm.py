"""GPU parity of the HIP LayerNorm (include/mvm_norm.h) against float64 torch
autograd through ``F.layer_norm`` on the CPU.

Tolerance per element: |got - ref| <= 1e-5 + 1e-4 * |ref| + 32 * 2^-24 * S,
where S is the float64 sum of the absolute values of the terms that make up
that element (so a float32 sum that cancels is held to its rounding, not to
the size of its result):
  y        S = |gamma| * rstd * (|x - mean| + mean_c |x|) + |beta|
  dx       S = rstd * (|g| + mean_c |g| + |xh| * mean_c |g * xh|) + |dres|
  dgamma   S = sum_r |dy * xh|        dbeta   S = sum_r |dy|
with g = dy * gamma and xh = (x - mean) * rstd.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

CANCEL = 32 * 2.0 ** -24


def _inputs(rows, cols, seed):
    g = torch.Generator().manual_seed(seed)
    x = 3.0 + 2.0 * torch.randn(rows, cols, generator=g)   # an offset mean: the variance pass matters
    w = 1.0 + 0.5 * torch.randn(cols, generator=g)
    b = 0.5 * torch.randn(cols, generator=g)
    dy = torch.randn(rows, cols, generator=g)
    dres = torch.randn(rows, cols, generator=g)
    return x, w, b, dy, dres


def _reference(x, w, b, dy, dres, eps):
    xd, wd, bd = [t.double().requires_grad_(True) for t in (x, w, b)]
    y = F.layer_norm(xd, (x.shape[-1],), wd, bd, eps)
    dx, dw, db = torch.autograd.grad(y, (xd, wd, bd), dy.double())
    dx = dx + dres.double()
    with torch.no_grad():
        xd = x.double()
        mu = xd.mean(-1, keepdim=True)
        r = 1.0 / torch.sqrt(((xd - mu) ** 2).mean(-1, keepdim=True) + eps)
        xh = (xd - mu) * r
        gg = dy.double() * w.double()
        s_y = w.double().abs() * r * ((xd - mu).abs() + xd.abs().mean(-1, keepdim=True)) + b.double().abs()
        s_dx = r * (gg.abs() + gg.abs().mean(-1, keepdim=True)
                    + xh.abs() * (gg * xh).abs().mean(-1, keepdim=True)) + dres.double().abs()
        s_dw = (dy.double() * xh).abs().sum(0)
        s_db = dy.double().abs().sum(0)
    return (y.detach(), dx, dw, db), (s_y, s_dx, s_dw, s_db)


def _close(name, got, ref, scale):
    got = got.detach().double().cpu()
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert torch.isfinite(got).all(), name
    err = (got - ref).abs()
    bound = 1e-5 + 1e-4 * ref.abs() + CANCEL * scale
    if err.numel() and bool((err > bound).any()):
        i = int(torch.argmax(err - bound))
        raise AssertionError(f"{name}: max err {float(err.max()):.3e}; worst flat index {i}: got "
                             f"{float(got.flatten()[i])}, ref {float(ref.flatten()[i])}")


def _run(cuda, x, w, b, dy, dres, eps, residual):
    from mlx_vision_mamba_amd.norm import _LayerNormFn
    xg, wg, bg = [t.to(cuda).requires_grad_(True) for t in (x, w, b)]
    if residual:
        y, xr = _LayerNormFn.apply(xg, wg, bg, eps, True)
        grads = torch.autograd.grad((y, xr), (xg, wg, bg), (dy.to(cuda), dres.to(cuda)))
    else:
        y = _LayerNormFn.apply(xg, wg, bg, eps, False)
        grads = torch.autograd.grad(y, (xg, wg, bg), dy.to(cuda))
    torch.cuda.synchronize()
    return (y,) + tuple(grads)


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 63), (100, 64), (6272, 384), (33, 1000),
                                       (5, 1024), (3000, 192), (9, 130)])
@pytest.mark.parametrize("residual", [False, True])
def test_layernorm_parity(cuda, rows, cols, residual):
    print(f"case: layernorm rows={rows} cols={cols} residual={residual}", flush=True)
    x, w, b, dy, dres = _inputs(rows, cols, seed=rows * 7 + cols)
    if not residual:
        dres = torch.zeros_like(dres)
    eps = 1e-5
    got = _run(cuda, x, w, b, dy, dres, eps, residual)
    refs, scales = _reference(x, w, b, dy, dres, eps)
    for name, g, r, s in zip(("y", "dx", "dgamma", "dbeta"), got, refs, scales):
        _close(name, g, r, s)


def test_layernorm_matches_torch_module_and_is_deterministic(cuda):
    """Against torch's own float32 LayerNorm on the GPU (same eps, weights),
    and bitwise repeatable."""
    from mlx_vision_mamba_amd.norm import layer_norm
    torch.manual_seed(3)
    norm = torch.nn.LayerNorm(384).to(cuda)
    with torch.no_grad():
        norm.weight.normal_(1.0, 0.3)
        norm.bias.normal_(0.0, 0.3)
    x = torch.randn(32, 196, 384, device=cuda)
    y1 = layer_norm(x, norm)
    y2 = layer_norm(x, norm)
    assert torch.equal(y1, y2)
    ref = norm(x)
    assert float((y1 - ref).detach().abs().max()) < 1e-5
    xg = x.clone().requires_grad_(True)
    g = torch.randn_like(x)
    a = torch.autograd.grad(layer_norm(xg, norm), [xg, norm.weight, norm.bias], g)
    c = torch.autograd.grad(layer_norm(xg, norm), [xg, norm.weight, norm.bias], g)
    for u, v in zip(a, c):
        assert torch.equal(u, v)


def test_layernorm_empty_rows(cuda):
    """No rows: an empty output and exact-zero dgamma / dbeta."""
    from mlx_vision_mamba_amd.norm import _LayerNormFn
    junk = [torch.full((64,), float("nan"), device=cuda) for _ in range(64)]
    del junk
    x = torch.randn(0, 64, device=cuda, requires_grad=True)
    w = torch.randn(64, device=cuda, requires_grad=True)
    b = torch.randn(64, device=cuda, requires_grad=True)
    y = _LayerNormFn.apply(x, w, b, 1e-5, False)
    assert y.shape == (0, 64)
    dx, dw, db = torch.autograd.grad(y, (x, w, b), torch.empty(0, 64, device=cuda))
    torch.cuda.synchronize()
    assert dx.shape == (0, 64)
    np.testing.assert_array_equal(dw.cpu().numpy(), 0)
    np.testing.assert_array_equal(db.cpu().numpy(), 0)
