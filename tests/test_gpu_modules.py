"""GPU parity of the module layer against the float64 functional restatement
of the reference (oracle/torch_ref.py), on identical weights and inputs.

The product modules run in float32 on the GPU (hipBLASLt GEMMs, the HIP
scan, index-remapped directions); the oracle runs the reference's
formulation in float64 on the CPU (materialised permutations, the scan
through the float64 oracle, torch autograd).  Tolerance per element for
the output and for the gradient of every parameter and of the input
(tests/module_bounds.py):
|got - ref| <= 1e-5 + 1e-4 |ref| + min(8 * 2^-24 * S, 1e-4 * max|ref|),
S the magnitude companion's sum of the magnitudes of the terms that form
the element with the errors of its factors (the running error analysis
oracle/torch_ref.py ``*_tc``).
"""

import pytest
import torch

import mlx_vision_mamba_amd as mvm
from oracle import torch_ref
from tests import module_bounds as mbd

pytestmark = pytest.mark.gpu


def _compare(name, got, ref, S=None, log=None):
    mbd.check(name, got, ref, S, log=log)


def _run_both(module, x, oracle_fn, device, tc_fn=None):
    """Module on the GPU against the float64 restatement ``oracle_fn`` (and
    its running error analysis ``tc_fn``, for the per-element bounds)."""
    torch.manual_seed(123)
    module = module.to(device)
    xg = x.to(device).requires_grad_(True)
    y = module(xg)
    gy = torch.randn(y.shape, generator=torch.Generator().manual_seed(7))
    y.backward(gy.to(device))
    params = torch_ref.params_from_module(module)
    xr = x.double().clone().requires_grad_(True)
    yr = oracle_fn(params, xr)
    yr.backward(gy.double())
    S = {}
    if tc_fn is not None:
        _, S = mbd.magnitudes(tc_fn, params, x.double(), gy.double())
    log = []
    _compare("output", y, yr, S.get("output"), log)
    _compare("input grad", xg.grad, xr.grad, S.get("input grad"), log)
    _compare_grads(module, params, S, log)
    if log:
        name, worst = max(log, key=lambda t: t[1])
        print(f"worst err / (2^-24 S) = {worst:.3f} ({name})", flush=True)


def _compare_grads(module, params, S=None, log=None):
    S = S or {}
    for n, p in module.named_parameters():
        if p.grad is None:   # not on the graph (e.g. patch_embed for token inputs)
            assert params[n].grad is None or not params[n].grad.any(), n
            continue
        _compare(f"grad {n}", p.grad, params[n].grad, S.get(f"grad {n}"), log)


def _mamba_mag(P, X):
    return torch_ref.mamba_block_tc(P, "", X, 16, 4)


def _dir_mag(K, grid, d_state=16):
    return lambda P, X: torch_ref.direction_block_tc(P, "", X, K, grid, d_state, 4)


@pytest.mark.parametrize("mode", ["sequential", "chunked", "hip", "metal_fused", "parallel",
                                  "metal_train"])
def test_mamba_block(cuda, mode):
    torch.manual_seed(0)
    blk = mvm.MambaBlock(d_model=32, d_state=16, scan_mode=mode)
    x = torch.randn(2, 40, 32)
    _run_both(blk, x, lambda p, xx: torch_ref.mamba_block(p, "", xx, 16, 4), cuda, _mamba_mag)


def test_residual_and_bidirectional(cuda):
    torch.manual_seed(1)
    blk = mvm.ResidualMambaBlock(d_model=32)
    x = torch.randn(2, 21, 32)

    def ref(p, xx):
        return xx + torch_ref.mamba_block(p, "mamba.", torch_ref.layer_norm(p, "norm.", xx), 16, 4)
    _run_both(blk, x, ref, cuda,
              lambda P, X: torch_ref.residual_block_tc(P, "", X, 16, 4))
    bi = mvm.BidirectionalMambaBlock(d_model=32)
    _run_both(bi, x, lambda p, xx: torch_ref.bidirectional_block(p, "", xx, 16, 4), cuda,
              lambda P, X: torch_ref.bidirectional_block_tc(P, "", X, 16, 4))


@pytest.mark.parametrize("K,grid,n", [(2, None, 13), (4, (4, 5), 20), (6, (2, 3, 2), 12),
                                      (8, (2, 2, 1, 3), 12), (4, (4, 5), 7)])
def test_multidirectional_block(cuda, K, grid, n):
    """n != prod(grid) exercises the K=2 fallback with blocks 0 and 1
    (mamba_block.py:554-559)."""
    torch.manual_seed(2)
    blk = mvm.MultiDirectionalMambaBlock(d_model=32, num_directions=K, grid_shape=grid)
    x = torch.randn(2, n, 32)
    _run_both(blk, x, lambda p, xx: torch_ref.direction_block(p, "", xx, K, grid, 16, 4), cuda,
              _dir_mag(K, grid))


@pytest.mark.parametrize("input_dim,shape,kw", [
    (2, (2, 32, 32, 1), {}),
    (3, (1, 16, 16, 16, 1), {}),
    (4, (1, 4, 16, 16, 16, 1), {"num_temporal_frames": 4, "temporal_patch_size": 2}),
])
def test_vision_mamba(cuda, input_dim, shape, kw):
    torch.manual_seed(3)
    model = mvm.VisionMamba(img_size=shape[-2], patch_size=8, embed_dim=32, depth=2,
                            input_dim=input_dim, **kw)
    x = torch.randn(*shape)

    common = dict(input_dim=input_dim, patch_size=8, depth=2, grid_shape=model.grid_shape,
                  d_state=16, d_conv=4, temporal_patch_size=kw.get("temporal_patch_size", 1))
    _run_both(model, x, lambda p, xx: torch_ref.vision_mamba(p, xx, **common), cuda,
              lambda P, X: torch_ref.vision_mamba_tc(P, X, **common))


def test_vision_mamba_patch_subset(cuda):
    """patch_indices selects a subset of tokens; the blocks then fall back
    to forward + backward scans (vision_mamba.py:214-216)."""
    torch.manual_seed(4)
    model = mvm.VisionMamba(img_size=32, patch_size=8, embed_dim=32, depth=2).to(cuda)
    idx = torch.tensor([0, 2, 3, 5, 8, 9, 15])
    x = torch.randn(2, len(idx), 32)

    def ref(p, xx):
        return torch_ref.vision_mamba(p, xx, input_dim=2, patch_size=8, depth=2,
                                      grid_shape=model.grid_shape, d_state=16, d_conv=4,
                                      patch_indices=idx)

    class Wrap(torch.nn.Module):
        def __init__(self, m):
            super().__init__()
            self.m = m

        def forward(self, xx):
            return self.m(xx, patch_indices=idx.to(xx.device))
    w = Wrap(model)
    torch.manual_seed(123)
    xg = x.to(cuda).requires_grad_(True)
    y = w(xg)
    gy = torch.randn(y.shape, generator=torch.Generator().manual_seed(7))
    y.backward(gy.to(cuda))
    params = torch_ref.params_from_module(model)
    xr = x.double().clone().requires_grad_(True)
    yr = ref(params, xr)
    yr.backward(gy.double())
    _, S = mbd.magnitudes(
        lambda P, X: torch_ref.vision_mamba_tc(
            P, X, input_dim=2, patch_size=8, depth=2, grid_shape=model.grid_shape,
            d_state=16, d_conv=4, patch_indices=idx), params, x.double(), gy.double())
    _compare("output", y, yr, S["output"])
    _compare("input grad", xg.grad, xr.grad, S["input grad"])
    _compare_grads(model, params, S)


def test_direction_block_small_state_ragged_channels(cuda):
    """d_state 8 (< 16 states per channel: padded lanes) and d_inner 48 (a
    partial 64-channel block) through the direction block."""
    torch.manual_seed(5)
    blk = mvm.MultiDirectionalMambaBlock(d_model=24, d_state=8, num_directions=4,
                                         grid_shape=(3, 4))
    x = torch.randn(3, 12, 24)
    _run_both(blk, x, lambda p, xx: torch_ref.direction_block(p, "", xx, 4, (3, 4), 8, 4), cuda,
              _dir_mag(4, (3, 4), 8))


def _train_steps(model, x, steps):
    opt = torch.optim.AdamW(model.parameters(), lr=1e-2, fused=True)
    for _ in range(steps):
        opt.zero_grad(set_to_none=True)
        model(x).square().mean().backward()
        opt.step()
    torch.cuda.synchronize()


def test_stacked_parameters_follow_optimizer_and_moves(cuda):
    """The direction blocks' parameters are slices of stacked buffers after
    the first forward: AdamW steps update them in place, so a fresh model
    loaded with the trained state dict computes the same output; moving the
    model off the GPU and back rebuilds the buffers from the current values."""
    torch.manual_seed(6)
    kw = dict(img_size=32, patch_size=8, embed_dim=32, depth=2, input_dim=2)
    model = mvm.VisionMamba(**kw).to(cuda)
    x = torch.randn(2, 32, 32, 1, generator=torch.Generator().manual_seed(8)).to(cuda)
    _train_steps(model, x, 3)
    with torch.no_grad():
        out = model(x)
    fresh = mvm.VisionMamba(**kw).to(cuda)
    fresh.load_state_dict(model.state_dict())
    with torch.no_grad():
        assert torch.equal(fresh(x), out)
    model.cpu()
    model.to(cuda)
    with torch.no_grad():
        assert torch.equal(model(x), out)
    # and training continues the same way on both copies (the patch
    # embedding's library convolution may sum its weight gradient in another
    # order, hence a tolerance)
    _train_steps(model, x, 2)
    _train_steps(fresh, x, 2)
    for (n, p), (_, q) in zip(model.named_parameters(), fresh.named_parameters()):
        assert torch.allclose(p, q, rtol=1e-4, atol=1e-6), n


def test_graph_captured_step_matches_eager(cuda):
    """The whole train step (forward, loss, backward, fused AdamW) captured
    in a HIP graph: each replay, with eager steps of a twin model and
    synchronisations between the replays, gives the twin's loss and
    parameters."""
    kw = dict(img_size=32, patch_size=8, embed_dim=32, depth=2, input_dim=2)

    def make():
        torch.manual_seed(9)
        m = mvm.VisionMamba(**kw).to(cuda)
        return m, torch.optim.AdamW(m.parameters(), lr=1e-2, fused=True, capturable=True)

    x = torch.randn(4, 32, 32, 1, generator=torch.Generator().manual_seed(10)).to(cuda)
    (mg, og), (me, oe) = make(), make()

    def step(m, o):
        o.zero_grad(set_to_none=True)
        loss = m(x).square().mean()
        loss.backward()
        o.step()
        return loss

    side = torch.cuda.Stream(cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):
        for _ in range(3):
            step(mg, og)
    torch.cuda.current_stream(cuda).wait_stream(side)
    for _ in range(3):
        step(me, oe)
    torch.cuda.synchronize()
    og.zero_grad(set_to_none=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gloss = mg(x).square().mean()
        gloss.backward()
        og.step()
    for i in range(5):
        g.replay()
        eloss = step(me, oe)
        torch.cuda.synchronize()
        assert torch.allclose(gloss.detach(), eloss.detach(), rtol=1e-6, atol=0), i
        for (n, p), (_, q) in zip(mg.named_parameters(), me.named_parameters()):
            assert torch.allclose(p, q, rtol=1e-5, atol=1e-7), (i, n)


def test_metal_mode_is_forward_only(cuda):
    """scan_mode "metal" is the reference's inference-only scan
    (mamba_metal.py:230): the output matches the oracle, and a backward
    reaches only out_proj (the block core is detached)."""
    torch.manual_seed(12)
    blk = mvm.MambaBlock(d_model=32, d_state=16, scan_mode="metal").to(cuda)
    x = torch.randn(2, 23, 32)
    y = blk(x.to(cuda))
    params = torch_ref.params_from_module(blk)
    with torch.no_grad():
        yr = torch_ref.mamba_block(params, "", x.double(), 16, 4)
    _, S = mbd.magnitudes(_mamba_mag, params, x.double(), torch.ones(yr.shape, dtype=torch.float64))
    _compare("output", y, yr, S["output"])
    y.sum().backward()
    assert blk.out_proj.weight.grad is not None
    for name in ("in_proj", "x_proj", "dt_proj", "conv1d"):
        assert getattr(blk, name).weight.grad is None, name
    assert blk.A_log.grad is None and blk.D.grad is None


def test_block_with_no_tokens(cuda):
    """A MambaBlock over an empty token axis: an empty output, and every
    parameter gradient (all of them sums over tokens) exactly zero."""
    print("case: MambaBlock with 0 tokens", flush=True)
    torch.manual_seed(5)
    blk = mvm.MambaBlock(d_model=32, d_state=16, scan_mode="metal_fused").to(cuda)
    x = torch.randn(2, 0, 32, device=cuda, requires_grad=True)
    # NaN garbage in the allocator: a gradient nobody writes would show
    junk = [torch.full((n,), float("nan"), device=cuda) for n in (64, 64 * 4, 64 * 16) for _ in range(64)]
    del junk
    y = blk(x)
    assert y.shape == (2, 0, 32)
    y.sum().backward()
    torch.cuda.synchronize()
    assert x.grad.shape == x.shape
    for name, p in blk.named_parameters():
        assert p.grad is not None, name
        assert torch.equal(p.grad, torch.zeros_like(p)), name
