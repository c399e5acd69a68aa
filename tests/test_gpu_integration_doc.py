"""The ctypes binding printed in the repository's integration guide (the
markdown file read below) runs as written.

The python block that starts with ``# hip_scan.py`` is executed (with the
library name replaced by the in-tree path) and its ``hip_selective_scan``
must give exactly the values and gradients of the package's own
``selective_scan`` (same kernels, same chunking, deterministic reductions).
"""

import os
import re

import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GUIDE = "INTEGRATION.md"  # the guide whose binding block is executed


def _stub_source():
    text = open(os.path.join(ROOT, GUIDE)).read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    src = [b for b in blocks if b.startswith("# hip_scan.py")]
    assert len(src) == 1, f"{GUIDE} must hold exactly one hip_scan.py block"
    return src[0]


def test_stub_is_present_and_names_the_library():
    src = _stub_source()
    assert 'ctypes.CDLL("libmvm_scan.so")' in src
    assert "def hip_selective_scan(x, delta, A, B, C, D)" in src


def test_stub_matches_package_scan(cuda):
    from mlx_vision_mamba_amd import _lib, selective_scan
    src = _stub_source().replace('ctypes.CDLL("libmvm_scan.so")', f"ctypes.CDLL({_lib.LIB_PATH!r})")
    ns = {}
    exec(compile(src, f"{GUIDE}:hip_scan.py", "exec"), ns)
    g = torch.Generator().manual_seed(7)
    B, L, D, N = 2, 100, 192, 16
    x = torch.randn(B, L, D, generator=g)
    dl = torch.nn.functional.softplus(torch.randn(B, L, D, generator=g) - 3)
    A = -torch.rand(D, N, generator=g) * 3 - 0.1
    Bm, Cm = torch.randn(B, L, N, generator=g), torch.randn(B, L, N, generator=g)
    Dv = torch.randn(D, generator=g)
    dy = torch.randn(B, L, D, generator=g).to(cuda)
    outs = []
    for fn in (ns["hip_selective_scan"], selective_scan):
        ins = [t.to(cuda).requires_grad_() for t in (x, dl, A, Bm, Cm, Dv)]
        y = fn(*ins)
        grads = torch.autograd.grad(y, ins, dy)
        outs.append([y.detach()] + [t.detach() for t in grads])
    for name, a, b in zip(("y", "du", "ddelta", "dA", "dB", "dC", "dD"), *outs):
        assert torch.equal(a, b), name
