"""GPU parity of the HIP selective scan against the float64 oracle.

Tolerance: |got - ref| <= 1e-5 + 1e-4 * |ref| elementwise, for the forward
output and the gradients du, dA, dB, dC, dD, whenever the kernel stores
float32.  With bfloat16 outputs the bar is the bf16 rounding of the stored
value: |got - ref| <= 1e-3 + 8e-3 * |ref|.

ddelta is a 16-term signed sum whose terms can be ~1e3 times larger than
the result; no float32 evaluation can then be within 1e-5 of the exact
value (the reference's own sequential algorithm run in float32 misses the
plain bar on this shape: max abs error 6.4e-5, worst err / (2^-24 S) = 14).
Its bound adds the cancellation term 32 * 2^-24 * S, where S is the
oracle's sum of the absolute values of those terms (oracle_ddelta_scale).
"""

import numpy as np
import pytest
import torch

from oracle import ref_lib, scan_oracle as so
from mlx_vision_mamba_amd import synthetic as scan_inputs

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-5, 1e-4
CANCEL = 32 * 2.0 ** -24
NAMES = ("du", "ddelta", "dA", "dB", "dC", "dD")


def assert_close(got, ref, name, atol=ATOL, rtol=RTOL, scale=None):
    got = got.detach().float().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{name}: non-finite values"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    if scale is not None:
        bound = bound + CANCEL * scale
        print(f"{name}: worst err / (2^-24 S) = {np.max(err / (2.0 ** -24 * scale + 1e-300)):.2f}")
    worst = np.max(err - bound) if err.size else -1
    if worst > 0:
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{name}: |got-ref| exceeds {atol}+{rtol}|ref| at {i}: got {got[i]}, "
                             f"ref {ref[i]}, max abs err {err.max():.3e}")


def run_scan(inputs, device, chunk_len=0, out_dtype=None):
    from mlx_vision_mamba_amd import scan
    u, dl, A, Bm, Cm, Dv, g = [t.to(device) for t in inputs]
    leaves = [t.clone().requires_grad_(True) for t in (u, dl, A, Bm, Cm, Dv)]
    y = scan.selective_scan(*leaves, chunk_len=chunk_len, out_dtype=out_dtype)
    grads = torch.autograd.grad(y, leaves, g.to(y.dtype))
    torch.cuda.synchronize()
    return y, grads


def run_raw(inputs, device, chunk_len=0, out_dtype=None):
    """Forward + VJP through the raw entry points (no autograd dtype casts),
    so that float32 outputs of bf16 inputs are seen as stored."""
    from mlx_vision_mamba_amd import scan
    u, dl, A, Bm, Cm, Dv, g = [t.to(device) for t in inputs]
    args = (u.unsqueeze(2), dl.unsqueeze(2), A.unsqueeze(0), Bm.unsqueeze(2), Cm.unsqueeze(2),
            Dv.unsqueeze(0))
    y, ck = scan.scan_forward(*args, chunk_len=chunk_len, out_dtype=out_dtype, save_ckpt=True)
    gr = scan.scan_backward(*args, g.unsqueeze(2), ckpt=ck, chunk_len=chunk_len, out_dtype=out_dtype)
    torch.cuda.synchronize()
    du, ddl, dA, dB, dC, dD = gr
    return y.squeeze(2), (du.squeeze(2), ddl.squeeze(2), dA[0], dB.squeeze(2), dC.squeeze(2), dD[0])


def oracle(inputs):
    u, dl, A, Bm, Cm, Dv, g = [t.float().numpy() for t in inputs]
    y = ref_lib.scan_fwd(u, dl, A, Bm, Cm, Dv)
    return y, ref_lib.scan_vjp(u, dl, A, Bm, Cm, Dv, g)


def ddelta_scale(inputs):
    u, dl, A, Bm, Cm, Dv, g = [t.float().numpy() for t in inputs]
    return ref_lib.ddelta_scale(u, dl, A, Bm, Cm, g)


def check_all(inputs, device, chunk_len=0, out_dtype=None, atol=ATOL, rtol=RTOL, raw=False):
    runner = run_raw if raw else run_scan
    y, grads = runner(inputs, device, chunk_len, out_dtype)
    y_ref, g_ref = oracle(inputs)
    scale = ddelta_scale(inputs)
    assert_close(y, y_ref, "y", atol, rtol)
    for name, a, b in zip(NAMES, grads, g_ref):
        assert_close(a, b, name, atol, rtol, scale=scale if name == "ddelta" else None)


def test_lane_layout_selftest(cuda):
    from mlx_vision_mamba_amd import scan
    out = scan.selftest_lanes(cuda).cpu().numpy()
    lanes = np.arange(64)
    np.testing.assert_array_equal(out[:64], 4 * (lanes & ~3) + 6)
    g, j = lanes & 3, (lanes >> 4) & 3
    np.testing.assert_array_equal(out[64:], 16000 * j + 480 + 16 * g)


def test_parity_single_block_shape(cuda):
    """B=2, L=196, d_inner=1536, N=16, fp32 (one MambaBlock's scan)."""
    print("case: B=2 L=196 D=1536 N=16 fp32 seed 0", flush=True)
    check_all(scan_inputs.make(2, 196, 1536, 16, seed=0), cuda)


# (1, 200, 64, 16): 7 chunks of 32 (carries folded in the main pass) and 13
# chunks of 16 (separate carry pass)
@pytest.mark.parametrize("shape", [(1, 1, 8, 16), (2, 17, 5, 5), (3, 50, 100, 13), (2, 64, 64, 16),
                                   (1, 33, 70, 1), (1, 200, 64, 16)])
@pytest.mark.parametrize("chunk_len", [0, 16, 32, "whole"])
def test_parity_shapes_and_chunkings(cuda, shape, chunk_len):
    print(f"case: shape={shape} chunk_len={chunk_len}", flush=True)
    check_all(scan_inputs.make(*shape, seed=3, a_mode="random"), cuda, chunk_len=chunk_len)


def test_dA_at_slow_decays_within_the_reference_precision(cuda):
    """dA where the decays are slow (random A = -exp(N(0,1)), so |A| delta
    reaches ~1e-4 and states and adjoints build up over hundreds of steps)
    at B=4, L=1000, D=3072: dA[d,n] sums 4000 terms lam delta e h that cancel
    to as little as 1e-5 of their magnitudes S (oracle_dA_scale).  No float32
    evaluation reaches the plain bar there: the reference's own sequential
    algorithm run in float32 (torch_ref.scan_sequential on the CPU, gradients
    by autograd) misses it on a few elements, with worst error ~55 * 2^-24 * S.
    The bound for dA is the plain bar plus 32 * 2^-24 * S for the default
    (chunked) call, as for ddelta, and, for the one-chunk call of the
    sequential mode (a single 1000-step recurrence per state, forward and
    backward, like the reference's own loop), the larger of that and 4 x the
    float32 reference algorithm's worst ratio on the same inputs."""
    from oracle import torch_ref
    print("case: dA at slow decays B=4 L=1000 D=3072 N=16", flush=True)
    inputs = scan_inputs.make(4, 1000, 3072, 16, seed=20, a_mode="random")
    npi = [t.float().numpy() for t in inputs]
    dA_ref = ref_lib.scan_vjp(*npi)[2]
    S = ref_lib.dA_scale(*npi[:5], npi[6])
    eps = 2.0 ** -24

    def ratio(got):
        err = np.abs(np.asarray(got, dtype=np.float64) - dA_ref)
        plain = int(np.sum(err > ATOL + RTOL * np.abs(dA_ref)))
        return float(np.max(err / (eps * S))), plain

    torch.set_num_threads(min(16, torch.get_num_threads()))
    leaves = [t.clone().requires_grad_(True) for t in inputs[:6]]
    y32 = torch_ref.scan_sequential(*leaves)
    dA32 = torch.autograd.grad(y32, leaves[2], inputs[6])[0].double().numpy()
    del y32, leaves
    r_ref, n_ref = ratio(dA32)
    _, grads = run_scan(inputs, cuda)
    r_def, n_def = ratio(grads[2].cpu().numpy())
    _, grads = run_scan(inputs, cuda, chunk_len="whole")
    r_seq, n_seq = ratio(grads[2].cpu().numpy())
    print(f"worst err / (2^-24 S), plain-bar misses: float32 reference {r_ref:.1f} ({n_ref}), "
          f"default {r_def:.1f} ({n_def}), one chunk {r_seq:.1f} ({n_seq})", flush=True)
    assert n_ref > 0          # the plain bar is out of reach of float32 here
    assert r_def <= 32
    assert r_seq <= max(32.0, 4 * r_ref)


def test_parity_long_sequence_many_chunks(cuda):
    print("case: B=2 L=4096 D=128 auto chunking", flush=True)
    check_all(scan_inputs.make(2, 4096, 128, 16, seed=4), cuda)


def test_parity_bf16_inputs_fp32_outputs(cuda):
    print("case: bf16 in, fp32 out, B=2 L=300 D=96", flush=True)
    inputs = scan_inputs.make(2, 300, 96, 16, seed=5, dtype=torch.bfloat16)
    check_all(inputs, cuda, out_dtype=torch.float32, raw=True)


def test_parity_bf16_outputs(cuda):
    print("case: bf16 in/out, B=2 L=300 D=96", flush=True)
    inputs = scan_inputs.make(2, 300, 96, 16, seed=6, dtype=torch.bfloat16)
    y, grads = run_scan(inputs, cuda)
    assert y.dtype == torch.bfloat16
    y_ref, g_ref = oracle(inputs)
    scale = ddelta_scale(inputs)
    assert_close(y, y_ref, "y", 1e-3, 8e-3)
    for name, a, b in zip(NAMES, grads, g_ref):
        if name in ("du", "dB", "dC"):
            assert_close(a, b, name, 1e-3, 8e-3)
        else:  # ddelta, dA, dD stay float32
            assert_close(a, b, name, scale=scale if name == "ddelta" else None)


def test_deterministic(cuda):
    inputs = scan_inputs.make(2, 500, 200, 16, seed=7)
    y1, g1 = run_scan(inputs, cuda)
    y2, g2 = run_scan(inputs, cuda)
    assert torch.equal(y1, y2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_backward_recomputes_checkpoints_when_not_saved(cuda):
    from mlx_vision_mamba_amd import scan
    u, dl, A, Bm, Cm, Dv, g = [t.to(cuda) for t in scan_inputs.make(2, 100, 64, 16, seed=8)]
    args = (u.unsqueeze(2), dl.unsqueeze(2), A.unsqueeze(0), Bm.unsqueeze(2), Cm.unsqueeze(2),
            Dv.unsqueeze(0))
    _, ck = scan.scan_forward(*args, save_ckpt=True)
    a = scan.scan_backward(*args, g.unsqueeze(2), ckpt=ck)
    b = scan.scan_backward(*args, g.unsqueeze(2), ckpt=None)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_strided_projection_views(cuda):
    """B and C as column slices of one (B, L, R+2N) projection, as in
    mamba_block.py:174-177; dB and dC come back with the same strides."""
    from mlx_vision_mamba_amd import scan
    u, dl, A, Bm, Cm, Dv, g = scan_inputs.make(2, 40, 32, 16, seed=9)
    big = torch.randn(2, 40, 7 + 32)
    big[..., 7:23] = Bm
    big[..., 23:] = Cm
    big = big.to(cuda).requires_grad_(True)
    leaves = [t.to(cuda).requires_grad_(True) for t in (u, dl, A, Dv)]
    y = scan.selective_scan(leaves[0], leaves[1], leaves[2], big[..., 7:23], big[..., 23:], leaves[3])
    gu, gd, gA, gbig, gD = torch.autograd.grad(y, leaves[:3] + [big, leaves[3]], g.to(cuda))
    y_ref, (du, ddl, dA, dB, dC, dD) = oracle((u, dl, A, Bm, Cm, Dv, g))
    assert_close(y, y_ref, "y")
    assert_close(gbig[..., 7:23], dB, "dB")
    assert_close(gbig[..., 23:], dC, "dC")
    assert_close(gbig[..., :7], np.zeros((2, 40, 7)), "unused columns")


@pytest.mark.parametrize("K,grid", [(2, (6, 7)), (4, (14, 14)), (6, (4, 3, 5)), (8, (2, 3, 2, 4))])
def test_direction_remap_parity(cuda, K, grid):
    """K index-remapped scans in one launch equal K oracle scans on the
    materialised permuted / reversed sequences (mamba_block.py:443-533)."""
    from mlx_vision_mamba_amd import scan
    print(f"case: directions K={K} grid={grid}", flush=True)
    L = int(np.prod(grid))
    bsz, D, N = 2, 48, 16
    gen = torch.Generator().manual_seed(10 + K)
    u = torch.randn(bsz, L, K, D, generator=gen)
    dl = torch.nn.functional.softplus(torch.randn(bsz, L, K, D, generator=gen) * 0.5 - 3.0)
    A = -torch.exp(torch.randn(K, D, N, generator=gen))
    Bm = torch.randn(bsz, L, K, N, generator=gen)
    Cm = torch.randn(bsz, L, K, N, generator=gen)
    Dv = torch.randn(K, D, generator=gen)
    g = torch.randn(bsz, L, K, D, generator=gen)
    tok = np.stack([so.seq_to_token(L, grid, *so.direction_axis_order(K, k)) for k in range(K)])
    tok_t = torch.tensor(tok, dtype=torch.int32, device=cuda)
    leaves = [t.to(cuda).requires_grad_(True) for t in (u, dl, A, Bm, Cm, Dv)]
    y = scan.selective_scan_directions(*leaves, seq_to_tok=tok_t)
    grads = torch.autograd.grad(y, leaves, g.to(cuda))
    for k in range(K):
        idx = tok[k]
        args = [u[:, idx, k], dl[:, idx, k], A[k], Bm[:, idx, k], Cm[:, idx, k], Dv[k], g[:, idx, k]]
        args = [a.numpy() for a in args]
        y_ref = ref_lib.scan_fwd(*args[:6])
        du, ddl, dA, dB, dC, dD = ref_lib.scan_vjp(*args)
        scale = ref_lib.ddelta_scale(args[0], args[1], args[2], args[3], args[4], args[6])
        assert_close(y[:, idx, k], y_ref, f"y[k={k}]")
        for name, got, ref in [("du", grads[0][:, idx, k], du), ("ddelta", grads[1][:, idx, k], ddl),
                               ("dA", grads[2][k], dA), ("dB", grads[3][:, idx, k], dB),
                               ("dC", grads[4][:, idx, k], dC), ("dD", grads[5][k], dD)]:
            assert_close(got, ref, f"{name}[k={k}]", scale=scale if name == "ddelta" else None)


def _host(t):
    return t.detach().float().cpu().numpy()


def test_parity_long_sequence_full_width(cuda):
    """B=8, L=16384, D=1536, N=16 with bf16 u/B/C/dy and automatic chunking
    (22 chunks of 752 positions: both aggregate passes and both carry
    kernels), against the oracle at full width, for both output
    instantiations: float32 outputs at the scan bar, bf16 outputs
    (y, du, dB, dC) at the bf16 bar.

    The oracle runs over channel slabs of 192 (each slab a complete
    oracle call).  y, du, ddelta, dA and dD are compared per slab; dB and dC
    are sums over all 1536 channels, so they are compared once, against
    the float64 sum of the slabs' dB and dC: the reduction over the 24
    channel blocks of the kernels is checked whole."""
    from mlx_vision_mamba_amd import scan
    bsz, L, D, N = 8, 16384, 1536, 16
    assert scan.chunk_len_for(bsz, L, D, N) == 752
    print("case: B=8 L=16384 D=1536 N=16 bf16 in, fp32 and bf16 out, full width", flush=True)
    inputs = scan_inputs.make(bsz, L, D, N, seed=11, dtype=torch.bfloat16)
    gpu = {}
    for name, odt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
        y, grads = run_raw(inputs, cuda, out_dtype=odt)
        assert y.dtype == odt and grads[0].dtype == odt and grads[3].dtype == odt
        assert grads[1].dtype == torch.float32 and grads[2].dtype == torch.float32
        gpu[name] = [_host(y)] + [_host(g) for g in grads]
        del y, grads
    torch.cuda.empty_cache()
    bars = {"f32": {n: (ATOL, RTOL) for n in ("y",) + NAMES},
            "bf16": {n: ((1e-3, 8e-3) if n in ("y", "du", "dB", "dC") else (ATOL, RTOL))
                     for n in ("y",) + NAMES}}
    u, dl, A, Bm, Cm, Dv, g = [t.float().numpy() for t in inputs]
    dB_ref = np.zeros((bsz, L, N))
    dC_ref = np.zeros((bsz, L, N))
    slab = 192
    for d0 in range(0, D, slab):
        sl = slice(d0, d0 + slab)
        cut = [np.ascontiguousarray(x[..., sl]) for x in (u, dl)]
        y_ref, (du, ddl, dA, dB, dC, dD), S = ref_lib.scan_all(
            cut[0], cut[1], A[sl], Bm, Cm, Dv[sl], np.ascontiguousarray(g[..., sl]))
        dB_ref += dB
        dC_ref += dC
        for name, got in gpu.items():
            for key, idx, ref in (("y", 0, y_ref), ("du", 1, du), ("ddelta", 2, ddl)):
                a, r = bars[name][key]
                assert_close(torch.from_numpy(got[idx][..., sl]), ref, f"{name} {key} [{d0}:]", a, r,
                             scale=S if key == "ddelta" else None)
            assert_close(torch.from_numpy(got[3][sl]), dA, f"{name} dA [{d0}:]")
            assert_close(torch.from_numpy(got[6][sl]), dD, f"{name} dD [{d0}:]")
        print(f"slab {d0}:{d0 + slab} ok", flush=True)
    for name, got in gpu.items():
        for key, idx, ref in (("dB", 4, dB_ref), ("dC", 5, dC_ref)):
            a, r = bars[name][key]
            assert_close(torch.from_numpy(got[idx]), ref, f"{name} {key}", a, r)


def test_full_long_sequence_properties(cuda):
    """B=8, L=16384, D=1536, N=16, bf16 u/B/C: too large for the oracle, so
    check properties that do not depend on size: bitwise determinism, and
    agreement of two different time-chunkings (two-pass carry vs longer
    chunks) within tolerance."""
    print("case: B=8 L=16384 D=1536 bf16 properties", flush=True)
    inputs = scan_inputs.make(8, 16384, 1536, 16, seed=12, dtype=torch.bfloat16)
    y1, g1 = run_raw(inputs, cuda, out_dtype=torch.float32)
    y2, g2 = run_raw(inputs, cuda, out_dtype=torch.float32)
    assert torch.equal(y1, y2) and all(torch.equal(a, b) for a, b in zip(g1, g2))
    del y2, g2
    y3, g3 = run_raw(inputs, cuda, chunk_len=4096, out_dtype=torch.float32)
    assert_close(y3, y1.cpu().double().numpy(), "y (chunk 4096 vs auto)")
    for name, a, b in zip(NAMES, g3, g1):
        assert_close(a, b.cpu().double().numpy(), f"{name} (chunk 4096 vs auto)", atol=1e-4, rtol=1e-3)


def _dirty_small_pool(device, numel, count=256):
    """Leave NaN-filled blocks of `numel` floats in the caching allocator so
    that an output the library fails to write reads back as NaN, not 0."""
    junk = [torch.full((numel,), float("nan"), device=device) for _ in range(count)]
    del junk


@pytest.mark.parametrize("bsz,L", [(0, 24), (2, 0)])
def test_empty_batch_or_sequence(cuda, bsz, L):
    """Sums over an empty (b, t) range: dA and dD come back as exact zeros,
    every other tensor is empty with its primal's shape."""
    from mlx_vision_mamba_amd import scan
    print(f"case: empty scan B={bsz} L={L}", flush=True)
    D, N = 32, 16
    u = torch.randn(bsz, L, D, device=cuda, requires_grad=True)
    dl = torch.rand(bsz, L, D, device=cuda, requires_grad=True)
    A = (-torch.arange(1, N + 1, dtype=torch.float32)).repeat(D, 1).to(cuda).requires_grad_(True)
    Bm = torch.randn(bsz, L, N, device=cuda, requires_grad=True)
    Cm = torch.randn(bsz, L, N, device=cuda, requires_grad=True)
    Dv = torch.ones(D, device=cuda, requires_grad=True)
    y = scan.selective_scan(u, dl, A, Bm, Cm, Dv)
    assert y.shape == (bsz, L, D)
    _dirty_small_pool(cuda, D * N)
    _dirty_small_pool(cuda, D)
    grads = torch.autograd.grad(y, [u, dl, A, Bm, Cm, Dv], torch.randn_like(y))
    torch.cuda.synchronize()
    for g, p in zip(grads, (u, dl, A, Bm, Cm, Dv)):
        assert g.shape == p.shape
    assert torch.equal(grads[2], torch.zeros_like(A))
    assert torch.equal(grads[5], torch.zeros_like(Dv))
