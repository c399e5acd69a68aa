"""GPU parity of the fused scan (softplus prologue + silu gate around the scan,
mamba_block.py:180-190) against the float64 oracle (scan_oracle.fused_*).

Layouts are those the direction blocks use: u and delta_raw direction-major
(K, B, N, D) in memory, z the second half of the in_proj output
(B, N, K, 2D), B / C column slices of the x_proj output (K, B*N, R + 2N),
y contiguous (B, N, K, D); outputs are written into views of the same kind.

Tolerance: |got - ref| <= 1e-5 + 1e-4 |ref| for y, du, dA, dB, dC, dD, dz.
The gradient of delta_raw is the scan's ddelta times sigmoid(x) and inherits
its cancellation term 32 * 2^-24 * S * sigmoid(x) (see test_gpu_scan.py);
the dt-bias gradient sums it over (b, t), so its bound adds the same term
summed over (b, t).
"""

import numpy as np
import pytest
import torch

from oracle import ref_lib, scan_oracle as so
from tests.test_gpu_scan import CANCEL, assert_close

pytestmark = pytest.mark.gpu


def _case(bsz, L, K, D, N, R, seed, grid=None, gate=True, bias=True):
    gen = torch.Generator().manual_seed(seed)
    u = torch.randn(K, bsz, L, D, generator=gen)
    draw = torch.randn(K, bsz, L, D, generator=gen) * 1.5 - 3.0
    draw[0, 0, 0, :4] = 22.0  # the linear branch of softplus
    b = torch.randn(K, D, generator=gen) * 0.5 if bias else None
    A = -torch.exp(torch.randn(K, D, N, generator=gen) * 0.5)
    dbc = torch.randn(K, bsz * L, R + 2 * N, generator=gen)
    Dv = torch.randn(K, D, generator=gen)
    xz = torch.randn(bsz, L, K, 2 * D, generator=gen) * 2.0
    g = torch.randn(bsz, L, K, D, generator=gen)
    if grid is not None:
        tok = np.stack([so.seq_to_token(L, grid, *so.direction_axis_order(K, k)) for k in range(K)])
    elif K == 2:
        tok = np.stack([np.arange(L), np.arange(L)[::-1]])
    else:
        tok = np.tile(np.arange(L), (K, 1))
    return dict(u=u, draw=draw, b=b, A=A, dbc=dbc, Dv=Dv, xz=xz, g=g, tok=tok.astype(np.int32),
                gate=gate, R=R, N=N)


def _bnkd(t, bsz, L):
    K, _, X = t.shape
    return t.view(K, bsz, L, X).permute(1, 2, 0, 3)


def _run_gpu(c, dev, chunk_len=0, a_is_log=False):
    from mlx_vision_mamba_amd import scan
    K, bsz, L, D = c["u"].shape
    R, N = c["R"], c["N"]
    u = c["u"].to(dev).view(K, bsz * L, D)
    draw = c["draw"].to(dev).view(K, bsz * L, D)
    dbc = c["dbc"].to(dev)
    xz = c["xz"].to(dev)
    z = xz[..., D:] if c["gate"] else None
    b = c["b"].to(dev) if c["b"] is not None else None
    A, Dv = c["A"].to(dev), c["Dv"].to(dev)
    if a_is_log:
        A = torch.log(-A)  # the kernels form A = -exp(A_log)
    tok = torch.tensor(c["tok"], device=dev)
    bc = _bnkd(dbc, bsz, L)
    args = (_bnkd(u, bsz, L), _bnkd(draw, bsz, L), b, A, bc[..., R:R + N], bc[..., R + N:], Dv, z)
    y, y_raw, ck = scan.scan_fused_forward(*args, tok=tok, chunk_len=chunk_len, save=True,
                                           a_is_log=a_is_log)
    dxz = torch.full_like(xz, float("nan"))
    d_dbc = torch.full_like(dbc, float("nan"))
    dd_v = _bnkd(d_dbc, bsz, L)
    out = scan.scan_fused_backward(*args, y_raw, ck, c["g"].to(dev), tok=tok, chunk_len=chunk_len,
                                   dB=dd_v[..., R:R + N], dC=dd_v[..., R + N:],
                                   dz=dxz[..., D:] if c["gate"] else None, a_is_log=a_is_log)
    torch.cuda.synchronize()
    return y, out, d_dbc, dxz


def _check(c, y, out, d_dbc, dxz, a_is_log=False):
    K, bsz, L, D = c["u"].shape
    R, N = c["R"], c["N"]
    du, ddr, db, dA, dB, dC, dD, dz = out
    bc = c["dbc"].view(K, bsz, L, R + 2 * N)
    zfull = c["xz"][..., D:]
    db_bound = np.zeros((K, D))
    for k in range(K):
        idx = c["tok"][k]
        uk, drk = c["u"][k][:, idx].numpy(), c["draw"][k][:, idx].numpy()
        bk = c["b"][k].numpy() if c["b"] is not None else None
        Bk, Ck = bc[k][:, idx, R:R + N].numpy(), bc[k][:, idx, R + N:].numpy()
        zk = zfull[:, idx, k].numpy() if c["gate"] else None
        gk = c["g"][:, idx, k].numpy()
        Ak, Dk = c["A"][k].numpy(), c["Dv"][k].numpy()
        y_ref, _, delta = so.fused_fwd(uk, drk, bk, Ak, Bk, Ck, Dk, zk)
        r = so.fused_vjp(uk, drk, bk, Ak, Bk, Ck, Dk, zk, gk)
        x = drk + (bk if bk is not None else 0.0)
        gs = gk * zk * so.sigmoid(zk) if c["gate"] else gk
        scale = ref_lib.ddelta_scale(uk, delta, Ak, Bk, Ck, gs) * so.sigmoid(x)
        db_bound[k] = CANCEL * scale.sum(axis=(0, 1))
        assert_close(y[:, idx, k], y_ref, f"y[k={k}]")
        assert_close(du[:, idx, k], r[0], f"du[k={k}]")
        assert_close(ddr[:, idx, k], r[1], f"ddelta_raw[k={k}]", scale=scale)
        # with A_log the kernels return dA_log = dA * A (chain rule of A = -exp(A_log))
        assert_close(dA[k], r[3] * Ak if a_is_log else r[3], f"dA[k={k}]")
        assert_close(dB[:, idx, k], r[4], f"dB[k={k}]")
        assert_close(dC[:, idx, k], r[5], f"dC[k={k}]")
        assert_close(dD[k], r[6], f"dD[k={k}]")
        if c["gate"]:
            assert_close(dz[:, idx, k], r[7], f"dz[k={k}]")
        if c["b"] is not None:
            ref_db = r[2]
            err = np.abs(db[k].cpu().numpy() - ref_db)
            assert np.all(err <= 1e-5 + 1e-4 * np.abs(ref_db) + db_bound[k]), f"dbias[k={k}]"
    # untouched columns of the shared gradient buffers keep their fill
    assert torch.isnan(d_dbc[..., :R]).all()
    if c["gate"]:
        assert torch.isnan(dxz[..., :D]).all() and not torch.isnan(dxz[..., D:]).any()


@pytest.mark.parametrize("K,grid,bsz,D", [(4, (14, 14), 2, 64), (2, None, 3, 40),
                                          (6, (4, 3, 5), 2, 24), (8, (2, 3, 2, 4), 1, 80)])
def test_fused_parity_directions(cuda, K, grid, bsz, D):
    L = int(np.prod(grid)) if grid else 37
    print(f"case: fused K={K} grid={grid} B={bsz} D={D} L={L}", flush=True)
    c = _case(bsz, L, K, D, 16, 7, seed=40 + K, grid=grid)
    _check(c, *_run_gpu(c, cuda))


@pytest.mark.parametrize("gate,bias", [(False, True), (True, False), (False, False)])
def test_fused_optional_gate_and_bias(cuda, gate, bias):
    print(f"case: fused gate={gate} bias={bias}", flush=True)
    c = _case(2, 50, 2, 48, 16, 5, seed=3, gate=gate, bias=bias)
    _check(c, *_run_gpu(c, cuda))


def test_fused_chunked_long_sequence(cuda):
    """Time chunks (the two-pass carry, with the softplus in every pass)."""
    print("case: fused chunked L=700 chunk=64", flush=True)
    c = _case(1, 700, 2, 64, 16, 4, seed=5)
    _check(c, *_run_gpu(c, cuda, chunk_len=64))


@pytest.mark.parametrize("chunk_len", [0, 64, 32])
def test_fused_a_log_parametrisation(cuda, chunk_len):
    """A passed as A_log (A = -exp(A_log) formed in the kernels): y and every
    gradient match the oracle, dA becoming dA * A, with one time chunk and
    with the two-pass carry (whose aggregate passes read A too): 5 chunks
    fold their carry in the main pass, 10 use the separate carry kernels."""
    print(f"case: fused A_log chunk_len={chunk_len}", flush=True)
    c = _case(1, 300, 4, 64, 16, 6, seed=9, grid=(15, 20))
    _check(c, *_run_gpu(c, cuda, chunk_len=chunk_len, a_is_log=True), a_is_log=True)


def test_fused_equals_unfused_composition(cuda):
    """Without gate and bias the fused call is softplus followed by the plain
    scan: it matches the plain HIP scan fed with torch's softplus(delta_raw)
    (equal up to the rounding of the two softplus evaluations)."""
    from mlx_vision_mamba_amd import scan
    c = _case(2, 64, 2, 64, 16, 6, seed=8, gate=False, bias=False)
    K, bsz, L, D = c["u"].shape
    y, out, _, _ = _run_gpu(c, cuda)
    u = _bnkd(c["u"].view(K, bsz * L, D), bsz, L).contiguous().to(cuda)
    delta = torch.nn.functional.softplus(_bnkd(c["draw"].view(K, bsz * L, D), bsz, L)).contiguous()
    bc = _bnkd(c["dbc"], bsz, L)
    y2, _ = scan.scan_forward(u, delta.to(cuda), c["A"].to(cuda), bc[..., 6:22].to(cuda),
                              bc[..., 22:].to(cuda), c["Dv"].to(cuda),
                              torch.tensor(c["tok"], device=cuda))
    torch.testing.assert_close(y, y2, rtol=1e-5, atol=1e-5)


def test_fused_64bit_row_offsets(cuda):
    """Row offsets beyond int32 inside one (batch, direction) slab (z and dz
    rows 2^25 floats apart, an 8.6 GB span) run the int64 instantiations of
    the kernels; they equal the int32 kernels on the same values bitwise."""
    from mlx_vision_mamba_amd import scan
    print("case: fused scan with z rows 2^25 floats apart (int64 offsets)", flush=True)
    bsz, L, K, D, N = 1, 65, 1, 64, 16
    gen = torch.Generator().manual_seed(77)
    u = torch.randn(bsz, L, K, D, generator=gen).to(cuda)
    draw = (torch.randn(bsz, L, K, D, generator=gen) - 3.0).to(cuda)
    bias = torch.randn(K, D, generator=gen).to(cuda) * 0.3
    A = -torch.exp(torch.randn(K, D, N, generator=gen) * 0.5).to(cuda)
    Bm = torch.randn(bsz, L, K, N, generator=gen).to(cuda)
    Cm = torch.randn(bsz, L, K, N, generator=gen).to(cuda)
    Dv = torch.randn(K, D, generator=gen).to(cuda)
    z = torch.randn(bsz, L, K, D, generator=gen).to(cuda)
    g = torch.randn(bsz, L, K, D, generator=gen).to(cuda)
    big = torch.empty(L, 1 << 25, device=cuda)
    zs = big[:, :D].view(bsz, L, K, D)        # row stride 2^25
    zs.copy_(z)
    assert zs.stride(1) == 1 << 25
    outs = []
    for zz in (z, zs):
        y, y_raw, ck = scan.scan_fused_forward(u, draw, bias, A, Bm, Cm, Dv, zz, save=True)
        grads = scan.scan_fused_backward(u, draw, bias, A, Bm, Cm, Dv, zz, y_raw, ck, g)
        outs.append([y] + [t for t in grads if t is not None])
        torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(*outs)):
        assert torch.equal(a, b.contiguous()), f"output {i}"
    del big
