"""The scan's C ABI driven from plain C.

tests/c_caller/scan_c_caller.c (built by __graft_entry__.build(), i.e.
`make -C tests/c_caller`) allocates with hipMalloc, validates, sizes the
checkpoints and workspace, runs mvm_scan_fwd and mvm_scan_bwd on its own HIP
stream, and writes its inputs and outputs to a file.  The outputs are checked
against the float64 oracle on those inputs at the scan parity bar of
tests/test_gpu_scan.py: |got - ref| <= 1e-5 + 1e-4 * |ref|, with dδ's
cancellation term 32 * 2^-24 * S.
"""

import os
import subprocess

import numpy as np
import pytest
import torch

from oracle import ref_lib
from tests.test_gpu_scan import NAMES, assert_close

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_caller", "scan_c_caller")


def _read(path):
    raw = open(path, "rb").read()
    B, L, D, N = (int(v) for v in np.frombuffer(raw[:32], dtype=np.int64))
    flat = np.frombuffer(raw[32:], dtype=np.float32)
    shapes = ([(B, L, D), (B, L, D), (D, N), (B, L, N), (B, L, N), (D,), (B, L, D)]
              + [(B, L, D), (B, L, D), (B, L, D), (D, N), (B, L, N), (B, L, N), (D,)])
    arrays, o = [], 0
    for s in shapes:
        n = int(np.prod(s))
        arrays.append(np.array(flat[o:o + n].reshape(s)))
        o += n
    assert o == flat.size, "unexpected file size"
    return (B, L, D, N), arrays[:7], arrays[7:]


def test_c_caller_matches_oracle(cuda, tmp_path):
    if not os.path.exists(EXE):
        raise RuntimeError(f"{EXE} is missing: build it with __graft_entry__.build() "
                           "(make -C tests/c_caller)")
    out = tmp_path / "scan_c_caller.bin"
    print("case: plain C caller, B=2 L=100 D=96 N=16 fp32, auto chunking", flush=True)
    run = subprocess.run([EXE, str(out)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    dims, ins, outs = _read(out)
    assert dims == (2, 100, 96, 16)
    u, dl, A, Bm, Cm, Dv, g = ins
    y_ref = ref_lib.scan_fwd(u, dl, A, Bm, Cm, Dv)
    grads_ref = ref_lib.scan_vjp(u, dl, A, Bm, Cm, Dv, g)
    scale = ref_lib.ddelta_scale(u, dl, A, Bm, Cm, g)
    assert_close(torch.from_numpy(outs[0]), y_ref, "y")
    for name, got, ref in zip(NAMES, outs[1:], grads_ref):
        assert_close(torch.from_numpy(got), ref, name, scale=scale if name == "ddelta" else None)
