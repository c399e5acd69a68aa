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


def _inputs(cuda, shape, seed):
    inputs = synthetic.make(*shape, seed=seed)
    u, dl, A, Bm, Cm, Dv, g = [t.to(cuda) for t in inputs]
    a4 = (u.unsqueeze(2), dl.unsqueeze(2), A.unsqueeze(0), Bm.unsqueeze(2), Cm.unsqueeze(2),
          Dv.unsqueeze(0))
    _, ck = scan.scan_forward(*a4, save_ckpt=True)
    ref = scan.scan_backward(*a4, g.unsqueeze(2), ckpt=ck)
    ref = (ref[0][:, :, 0], ref[1][:, :, 0], ref[2][0], ref[3][:, :, 0], ref[4][:, :, 0], ref[5][0])
    return (u, dl, A, Bm, Cm, Dv, ck, g), ref


def test_noalloc_backward_under_graph_capture(cuda):
    """mvm_scan_bwd_noalloc captured in a HIP graph (after an eager call on
    the device) and replayed: every replay, with eager work and
    synchronisations between the replays, is bitwise equal to mvm_scan_bwd."""
    print("case: mvm_scan_bwd_noalloc under graph capture", flush=True)
    args, ref = _inputs(cuda, (2, 196, 256, 16), 61)
    _noalloc_bwd(*args)          # eager call: the scratch address is resolved
    torch.cuda.synchronize()
    side = torch.cuda.Stream(cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):
        _noalloc_bwd(*args)
    torch.cuda.current_stream(cuda).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = _noalloc_bwd(*args)
    for i in range(4):
        graph.replay()
        junk = torch.randn(1 << 20, device=cuda) * 2   # eager work between replays
        torch.cuda.synchronize()
        for name, a, b in zip(NAMES, got, ref):
            assert torch.equal(a, b), (i, name)
        del junk


_FIRST_CALL_SCRIPT = r"""
import ctypes, sys, torch
sys.path.insert(0, {root!r})
from mlx_vision_mamba_amd import scan, synthetic
from tests.test_zz_no_alloc import _noalloc_bwd, NAMES
dev = torch.device("cuda:0")
inputs = synthetic.make(1, 100, 128, 16, seed=62)
u, dl, A, Bm, Cm, Dv, g = [t.to(dev) for t in inputs]
a4 = (u.unsqueeze(2), dl.unsqueeze(2), A.unsqueeze(0), Bm.unsqueeze(2), Cm.unsqueeze(2),
      Dv.unsqueeze(0))
_, ck = scan.scan_forward(*a4, save_ckpt=True)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):      # the process's first mvm_scan_bwd_noalloc call
    got = _noalloc_bwd(u, dl, A, Bm, Cm, Dv, ck, g)
ref = scan.scan_backward(*a4, g.unsqueeze(2), ckpt=ck)
ref = (ref[0][:, :, 0], ref[1][:, :, 0], ref[2][0], ref[3][:, :, 0], ref[4][:, :, 0], ref[5][0])
for i in range(3):
    graph.replay()
    torch.cuda.synchronize()
    for name, a, b in zip(NAMES, got, ref):
        assert torch.equal(a, b), (i, name)
print("FIRST_CALL_UNDER_CAPTURE_OK", flush=True)
"""


def test_noalloc_first_call_under_graph_capture(cuda):
    """The process's first mvm_scan_bwd_noalloc call made inside a graph
    capture (the call resolves the device's scratch address first): run in
    a fresh process, its replays equal mvm_scan_bwd bitwise."""
    import os
    import subprocess
    import sys
    print("case: mvm_scan_bwd_noalloc first call under capture (fresh process)", flush=True)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_SCRIPT.format(root=root)],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and "FIRST_CALL_UNDER_CAPTURE_OK" in res.stdout, \
        (res.returncode, res.stdout[-2000:], res.stderr[-4000:])
