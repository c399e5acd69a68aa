"""Seeded sweep of random shapes through the HIP scan and the fused scan,
each checked against the float64 oracle at the bars of test_gpu_scan.py and
test_gpu_fused.py.

The cases are drawn once from a fixed seed (the same cases every run):
batch 1-3, sequence 1-400, channels 1-300 (partial 64-channel blocks),
states 1-16, S4D-real or random decay rates, chunk lengths from none to
four tiles, float32 and bfloat16 inputs; fused cases add 1-4 directions
with random position tables, gate and dt bias on or off, and the A_log
parametrisation.  Each case prints its parameters before it runs.
"""

import numpy as np
import pytest

from mlx_vision_mamba_amd import synthetic as scan_inputs
from tests.test_gpu_fused import _case, _check, _run_gpu
from tests.test_gpu_scan import check_all

pytestmark = pytest.mark.gpu


def _scan_cases(n=24, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        B = int(rng.integers(1, 4))
        L = int(rng.integers(1, 401))
        D = int(rng.integers(1, 301))
        N = int(rng.integers(1, 17))
        chunk = [0, 16, 32, 48, 64, "whole"][int(rng.integers(0, 6))]
        bf16 = bool(rng.random() < 0.25)
        out.append((i, B, L, D, N, chunk, bf16))
    return out


@pytest.mark.parametrize("case", _scan_cases(), ids=lambda c: f"s{c[0]}")
def test_scan_random_shapes(cuda, case):
    import torch
    i, B, L, D, N, chunk, bf16 = case
    print(f"case: scan sweep {i}: B={B} L={L} D={D} N={N} chunk={chunk} bf16={bf16}", flush=True)
    dtype = torch.bfloat16 if bf16 else torch.float32
    inputs = scan_inputs.make(B, L, D, N, seed=1000 + i, dtype=dtype,
                              a_mode="random" if i % 2 else "s4d")
    if bf16:
        # bf16 inputs, float32 outputs through the raw entry points: the
        # stored gradients are float32, so the float32 bar applies
        check_all(inputs, cuda, chunk_len=chunk, out_dtype=torch.float32, raw=True)
    else:
        check_all(inputs, cuda, chunk_len=chunk)


def _fused_cases(n=12, seed=20261203):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        K = int(rng.integers(1, 5))
        B = int(rng.integers(1, 3))
        L = int(rng.integers(1, 160))
        D = int(rng.integers(1, 140))
        N = int(rng.integers(1, 17))
        R = int(rng.integers(1, 9))
        chunk = [0, 16, 32, 64][int(rng.integers(0, 4))]
        gate = bool(rng.random() < 0.7)
        bias = bool(rng.random() < 0.7)
        a_log = bool(rng.random() < 0.5)
        out.append((i, K, B, L, D, N, R, chunk, gate, bias, a_log))
    return out


@pytest.mark.parametrize("case", _fused_cases(), ids=lambda c: f"f{c[0]}")
def test_fused_random_shapes(cuda, case):
    i, K, B, L, D, N, R, chunk, gate, bias, a_log = case
    print(f"case: fused sweep {i}: K={K} B={B} L={L} D={D} N={N} R={R} chunk={chunk} "
          f"gate={gate} bias={bias} a_log={a_log}", flush=True)
    c = _case(B, L, K, D, N, R, seed=2000 + i, gate=gate, bias=bias)
    rng = np.random.default_rng(3000 + i)
    # an arbitrary permutation per direction (the kernels read through it)
    c["tok"] = np.stack([rng.permutation(L) for _ in range(K)]).astype(np.int32)
    y, out, d_dbc, dxz = _run_gpu(c, cuda, chunk_len=chunk, a_is_log=a_log)
    _check(c, y, out, d_dbc, dxz, a_is_log=a_log)
