"""GPU checks of the one-launch AdamW (include/mvm_optim.h) against
torch.optim.AdamW (foreach=False: the per-tensor reference loop) and a
float64 restatement of the update, over several steps.

Tolerance: rtol 1e-5 / atol 1e-7 against torch's float32 AdamW (the two
differ only in float32 rounding order: fused multiply-adds and the
division); against the float64 restatement, float32's rounding of p and of
each update over the steps taken (see the bound in the test).
"""

import math

import pytest
import torch

from mlx_vision_mamba_amd.optim import AdamW

pytestmark = pytest.mark.gpu

SHAPES = [(1,), (3,), (2047,), (2048,), (2049,), (7, 11), (64, 33), (5000,), (0,)]


def _params(shapes, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return [torch.nn.Parameter(torch.randn(*s, generator=g).to(dev)) for s in shapes]


def _grads(params, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(p.shape, generator=g).to(p.device) for p in params]


def _adamw64(p, grads, steps, lr, b1, b2, eps, wd):
    """float64 AdamW: p <- p(1 - lr wd); m, v moments; bias-corrected step."""
    p = p.double().clone()
    m = torch.zeros_like(p)
    v = torch.zeros_like(p)
    for t in range(1, steps + 1):
        g = grads[t - 1].double()
        p = p * (1 - lr * wd)
        m = m + (1 - b1) * (g - m)
        v = b2 * v + (1 - b2) * g * g
        denom = v.sqrt() / math.sqrt(1 - b2 ** t) + eps
        p = p - lr / (1 - b1 ** t) * m / denom
    return p


@pytest.mark.parametrize("wd", [0.0, 0.05])
def test_adamw_matches_torch_and_float64(cuda, wd):
    print("case: AdamW vs torch.optim.AdamW, shapes", SHAPES, "wd", wd, flush=True)
    ours = _params(SHAPES, 0, cuda)
    ref = [torch.nn.Parameter(p.detach().clone()) for p in ours]
    start = [p.detach().clone() for p in ours]
    kw = dict(lr=3e-3, betas=(0.9, 0.99), eps=1e-8, weight_decay=wd)
    opt = AdamW(ours, **kw)
    ropt = torch.optim.AdamW(ref, foreach=False, **kw)
    history = []
    for step in range(5):
        gs = _grads(ours, 100 + step)
        history.append(gs)
        for p, r, g in zip(ours, ref, gs):
            p.grad = g.clone()
            r.grad = g.clone()
        opt.step()
        ropt.step()
        torch.cuda.synchronize()
        for p, r in zip(ours, ref):
            torch.testing.assert_close(p.detach(), r.detach(), rtol=1e-5, atol=1e-7)
    for i, p in enumerate(ours):
        want = _adamw64(start[i], [h[i] for h in history], 5, 3e-3, 0.9, 0.99, 1e-8, wd)
        err = (p.detach().double() - want).abs()
        # float32 rounds p (2^-24 |p|) and each update (~lr 2^-22) at every step
        bound = 5 * (2.0 ** -24 * want.abs() + 3e-3 * 2.0 ** -20) + 1e-7 * want.abs()
        assert (err <= bound).all(), (SHAPES[i], (err / bound).max().item())


def test_adamw_many_tensors_and_missing_grads(cuda):
    """More tensors than one launch's table holds; tensors without a gradient
    keep their values and moments."""
    print("case: AdamW over 150 tensors, every 7th without a gradient", flush=True)
    shapes = [(1 + (37 * i) % 300,) for i in range(150)]
    ours = _params(shapes, 1, cuda)
    ref = [torch.nn.Parameter(p.detach().clone()) for p in ours]
    opt = AdamW(ours, lr=1e-3)
    ropt = torch.optim.AdamW(ref, lr=1e-3, foreach=False)
    for step in range(3):
        gs = _grads(ours, 200 + step)
        for i, (p, r, g) in enumerate(zip(ours, ref, gs)):
            p.grad = None if i % 7 == 0 else g.clone()
            r.grad = None if i % 7 == 0 else g.clone()
        opt.step()
        ropt.step()
    torch.cuda.synchronize()
    for p, r in zip(ours, ref):
        torch.testing.assert_close(p.detach(), r.detach(), rtol=1e-5, atol=1e-7)
    for i in range(0, 150, 7):
        off, n = opt.offsets[i], ours[i].numel()
        assert torch.equal(opt.exp_avg[off:off + n], torch.zeros(n, device=cuda))


def test_adamw_graph_replays(cuda):
    """The step captured in a HIP graph: each replay (with eager work and a
    synchronisation in between) matches the same number of eager steps."""
    print("case: AdamW captured in a graph, 3 replays", flush=True)
    shapes = [(300,), (17, 5), (2049,)]
    cap = _params(shapes, 2, cuda)
    eag = [torch.nn.Parameter(p.detach().clone()) for p in cap]
    gs = _grads(cap, 300)
    for p, e, g in zip(cap, eag, gs):
        p.grad = g.clone()
        e.grad = g.clone()
    opt, eopt = AdamW(cap, lr=2e-3), AdamW(eag, lr=2e-3)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        opt.step()
    for replay in range(3):
        graph.replay()
        eopt.step()
        junk = torch.randn(1000, device=cuda).sum()  # eager work between replays
        torch.cuda.synchronize()
        assert float(opt.step_count) == replay + 1 == float(eopt.step_count)
        for p, e in zip(cap, eag):
            assert torch.equal(p.detach(), e.detach()), replay
        del junk
