"""The drop-in surface, on the GPU.

* The reference's scan entry points under their own names
  (mamba_block.py:20 ``selective_scan``; mamba_fast.py:17, :165
  ``selective_scan_chunked`` / ``_parallel``; mamba_metal.py:230, :275
  ``selective_scan_metal`` / ``_metal_trainable``; mamba_metal_fused.py:253
  ``selective_scan_metal_fused``) at B=2, L=196, D=1536, N=16 against the
  float64 C oracle, at the scan bar (ddelta widened by 32 * 2^-24 * S).
* ``MambaBlock._scan_fn`` (mamba_block.py:104-122, called at :187): a
  replaced scan function is called with the reference's arguments, in a
  single block and inside direction blocks, and gives the oracle's result.
* Layout and mode corner cases: B and C broadcast over the batch, no_grad
  forwards, malformed direction tables.
* Module parity at a real layer width: one MultiDirectionalMambaBlock of
  the VisionMamba-2D encoder (E=384, d_inner=768, K=4, 14x14 grid), of the
  3D encoder (K=6, 16^3 grid) and of the 4D encoder (K=8, grid
  (8, 4, 4, 4)), against the float64 restatement, at the per-element
  module bound (tests/module_bounds.py).
"""

import numpy as np
import pytest
import torch

import mlx_vision_mamba_amd as mvm
from mlx_vision_mamba_amd import synthetic
from oracle import ref_lib, torch_ref
from tests.test_gpu_modules import _compare, _dir_mag, _mamba_mag, _run_both
from tests.test_gpu_scan import NAMES, assert_close, ddelta_scale, oracle

pytestmark = pytest.mark.gpu

ENTRY_POINTS = ["selective_scan", "selective_scan_sequential", "selective_scan_chunked",
                "selective_scan_parallel", "selective_scan_metal_trainable",
                "selective_scan_metal_fused"]


@pytest.fixture(scope="module")
def single_block():
    """One MambaBlock's scan: B=2, L=196, d_inner=1536, N=16, fp32, with its oracle results."""
    inputs = synthetic.make(2, 196, 1536, 16, seed=0)
    return inputs, oracle(inputs), ddelta_scale(inputs)


@pytest.mark.parametrize("name", ENTRY_POINTS)
def test_entry_point_matches_oracle(cuda, single_block, name):
    print(f"case: {name} at B=2 L=196 D=1536 N=16", flush=True)
    inputs, (y_ref, g_ref), scale = single_block
    fn = getattr(mvm, name)
    leaves = [t.to(cuda).requires_grad_(True) for t in inputs[:6]]
    y = fn(*leaves)
    grads = torch.autograd.grad(y, leaves, inputs[6].to(cuda))
    assert_close(y, y_ref, f"{name} y")
    for n, a, b in zip(NAMES, grads, g_ref):
        assert_close(a, b, f"{name} {n}", scale=scale if n == "ddelta" else None)


def test_metal_entry_point_is_forward_only(cuda, single_block):
    inputs, (y_ref, _), _ = single_block
    leaves = [t.to(cuda).requires_grad_(True) for t in inputs[:6]]
    y = mvm.selective_scan_metal(*leaves)
    assert not y.requires_grad
    assert_close(y, y_ref, "selective_scan_metal y")


def test_scan_mode_registry_returns_the_entry_points():
    for mode, name in [("sequential", "selective_scan_sequential"),
                       ("chunked", "selective_scan_chunked"),
                       ("parallel", "selective_scan_parallel"), ("metal", "selective_scan_metal"),
                       ("metal_train", "selective_scan_metal_trainable"),
                       ("metal_fused", "selective_scan_metal_fused"), ("hip", "selective_scan")]:
        assert mvm.get_scan_fn(mode) is getattr(mvm, name)
        assert mvm.MambaBlock(16, scan_mode=mode)._scan_fn is getattr(mvm, name)


class _Recorder:
    """A replacement scan function: the library's sequential scan, with its
    calls and argument shapes recorded."""

    def __init__(self):
        self.shapes = []

    def __call__(self, x, delta, A, B, C, D):
        self.shapes.append(tuple(tuple(t.shape) for t in (x, delta, A, B, C, D)))
        return mvm.selective_scan_sequential(x, delta, A, B, C, D)


def test_replaced_scan_fn_is_called_in_a_block(cuda):
    torch.manual_seed(0)
    blk = mvm.MambaBlock(d_model=32, d_state=16)
    rec = _Recorder()
    blk._scan_fn = rec
    x = torch.randn(2, 40, 32)
    _run_both(blk, x, lambda p, xx: torch_ref.mamba_block(p, "", xx, 16, 4), cuda, _mamba_mag)
    assert rec.shapes == [((2, 40, 64), (2, 40, 64), (64, 16), (2, 40, 16), (2, 40, 16), (64,))]


def test_replaced_scan_fn_in_direction_blocks(cuda):
    """Each direction's own block (and scan function) runs on its scan
    order, as in mamba_block.py:407-566."""
    torch.manual_seed(1)
    K, grid = 4, (4, 5)
    blk = mvm.MultiDirectionalMambaBlock(d_model=32, num_directions=K, grid_shape=grid)
    recs = []
    for b in blk.mamba_blocks:
        recs.append(_Recorder())
        b._scan_fn = recs[-1]
    x = torch.randn(2, 20, 32)
    _run_both(blk, x, lambda p, xx: torch_ref.direction_block(p, "", xx, K, grid, 16, 4), cuda,
              _dir_mag(K, grid))
    assert all(len(r.shapes) == 1 for r in recs)
    bi = mvm.BidirectionalMambaBlock(d_model=32)
    bi.backward_mamba._scan_fn = _Recorder()
    _run_both(bi, x, lambda p, xx: torch_ref.bidirectional_block(p, "", xx, 16, 4), cuda,
              lambda P, X: torch_ref.bidirectional_block_tc(P, "", X, 16, 4))
    assert len(bi.backward_mamba._scan_fn.shapes) == 1


def test_broadcast_B_and_C_over_batch(cuda):
    """B and C expanded over the batch (stride 0): dB and dC are the sums of
    the per-batch gradients, as autograd of the expand gives."""
    inputs = synthetic.make(3, 50, 40, 16, seed=21)
    u, dl, A, Bm, Cm, Dv, g = inputs
    B1, C1 = Bm[:1], Cm[:1]
    leaves = [t.to(cuda).requires_grad_(True) for t in (u, dl, A, B1, C1, Dv)]
    y = mvm.selective_scan(leaves[0], leaves[1], leaves[2], leaves[3].expand(3, -1, -1),
                           leaves[4].expand(3, -1, -1), leaves[5])
    grads = torch.autograd.grad(y, leaves, g.to(cuda))
    Bx, Cx = B1.expand(3, -1, -1).contiguous(), C1.expand(3, -1, -1).contiguous()
    y_ref, (du, ddl, dA, dB, dC, dD) = oracle((u, dl, A, Bx, Cx, Dv, g))
    assert_close(y, y_ref, "y")
    assert_close(grads[3], dB.sum(0, keepdims=True), "dB summed over batch")
    assert_close(grads[4], dC.sum(0, keepdims=True), "dC summed over batch")
    assert_close(grads[0], du, "du")


def test_no_grad_forward_equals_training_forward(cuda):
    torch.manual_seed(2)
    model = mvm.VisionMamba(img_size=32, patch_size=8, embed_dim=32, depth=2).to(cuda)
    x = torch.randn(2, 32, 32, 1, device=cuda)
    y_train = model(x)
    with torch.no_grad():
        y_eval = model(x)
    with torch.inference_mode():
        y_inf = model(x)
    assert torch.equal(y_train.detach(), y_eval) and torch.equal(y_eval, y_inf)
    y_train.sum().backward()       # the training forward still saved its state
    assert all(p.grad is not None for p in model.blocks.parameters())


def test_malformed_direction_table_rejected(cuda):
    u = torch.randn(1, 6, 2, 16, device=cuda)
    A = -torch.ones(2, 16, 4, device=cuda)
    Bm = torch.randn(1, 6, 2, 4, device=cuda)
    Dv = torch.ones(2, 16, device=cuda)
    good = torch.tensor([[0, 1, 2, 3, 4, 5], [5, 4, 3, 2, 1, 0]], dtype=torch.int32, device=cuda)
    mvm.selective_scan_directions(u, u.abs(), A, Bm, Bm, Dv, seq_to_tok=good)
    bad = torch.tensor([[0, 1, 2, 3, 4, 4], [5, 4, 3, 2, 1, 0]], dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError, match="permutation"):
        mvm.selective_scan_directions(u, u.abs(), A, Bm, Bm, Dv, seq_to_tok=bad)
    good[0, 5] = 4           # an in-place change is checked again
    with pytest.raises(ValueError, match="permutation"):
        mvm.selective_scan_directions(u, u.abs(), A, Bm, Bm, Dv, seq_to_tok=good)


@pytest.mark.parametrize("K,grid,bsz", [(4, (14, 14), 2), (6, (16, 16, 16), 1), (8, (8, 4, 4, 4), 1)])
def test_direction_block_at_layer_width(cuda, K, grid, bsz):
    """One encoder layer at its real width (E=384, d_inner=768, N=16):
    the VisionMamba-2D layer (K=4, 14x14 grid), the 3D layer (K=6, 16^3
    grid, L=4096: at batch 1 the fused scan runs 52 time chunks of 80
    positions, joined by the separate carry kernels) and the 4D layer (K=8, grid (8, 4, 4, 4), L=512), output and
    every gradient against the float64 restatement (mamba_block.py:407-566;
    its scan is the float64 C oracle, torch_ref.scan_oracle_c)."""
    from mlx_vision_mamba_amd import scan
    print(f"case: direction block E=384 K={K} grid={grid} batch={bsz}", flush=True)
    L = int(np.prod(grid))
    if K == 6:
        assert -(-L // scan.chunk_len_for(bsz * K, L, 768)) > 8   # the carry kernels run
    torch.manual_seed(5 + K)
    blk = mvm.MultiDirectionalMambaBlock(d_model=384, num_directions=K, grid_shape=grid)
    x = torch.randn(bsz, L, 384)
    _run_both(blk, x, lambda p, xx: torch_ref.direction_block(p, "", xx, K, grid, 16, 4,
                                                              scan=torch_ref.scan_oracle_c), cuda,
              _dir_mag(K, grid))
