"""mvm_scan_bwd_noalloc (the backward that takes its scratch from the
library's static per-GPU array instead of a workspace) against
mvm_scan_bwd, through the C ABI: two calls in a row, the second on a
smaller input, each bitwise equal to mvm_scan_bwd's result and within the
scan bar of the float64 oracle."""

import ctypes

import pytest
import torch

from mlx_vision_mamba_amd import _lib, scan, synthetic
from tests.test_gpu_scan import NAMES, assert_close, ddelta_scale, oracle

pytestmark = pytest.mark.gpu


def _noalloc_bwd(u, dl, A, Bm, Cm, Dv, ck, g):
    """Calls mvm_scan_bwd_noalloc on (B, L, D) inputs (one direction)."""
    args = [t.unsqueeze(2) for t in (u, dl)] + [A.unsqueeze(0), Bm.unsqueeze(2), Cm.unsqueeze(2),
                                               Dv.unsqueeze(0)]
    u4, dl4, A3, B4, C4, D2 = args
    desc = scan._make_desc(u4, B4, torch.float32, torch.float32, None, 0)
    du = torch.full_like(u4, float("nan"))
    ddl = torch.full_like(u4, float("nan"))
    dA = torch.full_like(A3, float("nan"))
    dB = torch.full_like(B4, float("nan"))
    dC = torch.full_like(B4, float("nan"))
    dD = torch.full_like(D2, float("nan"))
    g4 = g.unsqueeze(2).contiguous()
    with torch.cuda.device(u.device):
        _lib.check(_lib.lib().mvm_scan_bwd_noalloc(
            ctypes.byref(desc), *[scan._ptr(t) for t in (u4, dl4, A3, B4, C4, D2, ck, g4, du, ddl,
                                                         dA, dB, dC, dD)],
            ctypes.c_void_p(scan._stream_ptr(u.device))))
    return du[:, :, 0], ddl[:, :, 0], dA[0], dB[:, :, 0], dC[:, :, 0], dD[0]


@pytest.mark.parametrize("shape", [(2, 196, 1536, 16), (1, 50, 72, 8)])
def test_noalloc_backward_equals_workspace_backward(cuda, shape):
    print(f"case: mvm_scan_bwd_noalloc shape={shape}", flush=True)
    inputs = synthetic.make(*shape, seed=60)
    u, dl, A, Bm, Cm, Dv, g = [t.to(cuda) for t in inputs]
    a4 = (u.unsqueeze(2), dl.unsqueeze(2), A.unsqueeze(0), Bm.unsqueeze(2), Cm.unsqueeze(2),
          Dv.unsqueeze(0))
    _, ck = scan.scan_forward(*a4, save_ckpt=True)
    ref = scan.scan_backward(*a4, g.unsqueeze(2), ckpt=ck)
    ref = (ref[0][:, :, 0], ref[1][:, :, 0], ref[2][0], ref[3][:, :, 0], ref[4][:, :, 0], ref[5][0])
    got = _noalloc_bwd(u, dl, A, Bm, Cm, Dv, ck, g)
    torch.cuda.synchronize()
    for name, a, b in zip(NAMES, got, ref):
        assert torch.equal(a, b), name
    _, g_ref = oracle(inputs)
    scale = ddelta_scale(inputs)
    for name, a, b in zip(NAMES, got, g_ref):
        assert_close(a, b, name, scale=scale if name == "ddelta" else None)
