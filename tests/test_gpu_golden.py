"""The HIP path against the committed golden fixtures (tests/golden/):
the plain scan and the fused block prologue / epilogue, forward and VJP,
at the scan bar |got - ref| <= 1e-5 + 1e-4 |ref| (ddelta and the gradient
of delta_raw widened by their cancellation term, see test_gpu_scan.py)."""

import numpy as np
import pytest
import torch

from tests.test_golden import load
from tests.test_gpu_scan import CANCEL, NAMES, assert_close

pytestmark = pytest.mark.gpu


def test_scan_against_fixture(cuda):
    from mlx_vision_mamba_amd import scan
    f = load("scan_small.npz")
    ins = [torch.from_numpy(f[k]).to(cuda) for k in ("u", "delta", "A", "B", "C", "D")]
    leaves = [t.clone().requires_grad_(True) for t in ins]
    y = scan.selective_scan(*leaves)
    grads = torch.autograd.grad(y, leaves, torch.from_numpy(f["g"]).to(cuda))
    assert_close(y, f["y"], "y")
    for name, got in zip(NAMES, grads):
        assert_close(got, f[name], name, scale=f["S"] if name == "ddelta" else None)


def test_fused_against_fixture(cuda):
    from mlx_vision_mamba_amd import scan
    f = load("fused_small.npz")
    t = {k: torch.from_numpy(f[k]).to(cuda) for k in ("u", "delta_raw", "bias", "A", "B", "C",
                                                        "D", "z", "g")}
    u, draw, z, g = (t[k].unsqueeze(2) for k in ("u", "delta_raw", "z", "g"))
    Bm, Cm = t["B"].unsqueeze(2), t["C"].unsqueeze(2)
    A, Dv, bias = t["A"].unsqueeze(0), t["D"].unsqueeze(0), t["bias"].unsqueeze(0)
    y, y_raw, ck = scan.scan_fused_forward(u, draw, bias, A, Bm, Cm, Dv, z, save=True)
    out = scan.scan_fused_backward(u, draw, bias, A, Bm, Cm, Dv, z, y_raw, ck, g)
    du, ddr, db, dA, dB, dC, dD, dz = out
    assert_close(y[:, :, 0], f["y"], "y")
    assert_close(y_raw[:, :, 0], f["y_raw"], "y_raw")
    for name, got, ref in [("du", du, f["du"]), ("dA", dA[0], f["dA"]), ("dB", dB, f["dB"]),
                           ("dC", dC, f["dC"]), ("dD", dD[0], f["dD"]), ("dz", dz, f["dz"])]:
        assert_close(got.squeeze(2) if got.dim() == 4 else got, ref, name)
    # the delta_raw gradient carries the cancellation term of ddelta times
    # sigmoid(x) (S_raw); the dt-bias gradient sums it over (b, t)
    assert_close(ddr[:, :, 0], f["ddelta_raw"], "ddelta_raw", scale=f["S_raw"])
    err = np.abs(db[0].cpu().numpy() - f["dbias"])
    bound = 1e-5 + 1e-4 * np.abs(f["dbias"]) + CANCEL * f["S_raw"].sum(axis=(0, 1))
    assert np.all(err <= bound), "dbias"
