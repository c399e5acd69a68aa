"""The committed golden fixtures (tests/golden/, written by
tests/golden/make_golden.py from the pinned oracle): the oracle still
reproduces them, and the product's direction tables equal them."""

import os

import numpy as np

from mlx_vision_mamba_amd import directions as dirs
from oracle import ref_lib, scan_oracle as so

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_scan_fixture_reproduced_by_oracle():
    f = load("scan_small.npz")
    ins = [f[k] for k in ("u", "delta", "A", "B", "C", "D", "g")]
    assert all(a.dtype == np.float32 for a in ins)
    np.testing.assert_allclose(ref_lib.scan_fwd(*ins[:6]), f["y"], rtol=1e-13, atol=1e-14)
    for name, got in zip(("du", "ddelta", "dA", "dB", "dC", "dD"), ref_lib.scan_vjp(*ins)):
        np.testing.assert_allclose(got, f[name], rtol=1e-12, atol=1e-13, err_msg=name)
    np.testing.assert_allclose(so.scan_fwd(*ins[:6]), f["y"], rtol=1e-12, atol=1e-13)


def test_fused_fixture_reproduced_by_oracle():
    f = load("fused_small.npz")
    ins = [f[k].astype(np.float64) for k in ("u", "delta_raw", "bias", "A", "B", "C", "D", "z", "g")]
    y, y_raw, _ = so.fused_fwd(*ins[:8])
    np.testing.assert_allclose(y, f["y"], rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(y_raw, f["y_raw"], rtol=1e-13, atol=1e-14)
    names = ("du", "ddelta_raw", "dbias", "dA", "dB", "dC", "dD", "dz")
    for name, got in zip(names, so.fused_vjp(*ins)):
        np.testing.assert_allclose(got, f[name], rtol=1e-12, atol=1e-13, err_msg=name)


def test_direction_tables_equal_fixture():
    f = load("directions.npz")
    for K, grid in ((4, (3, 4)), (6, (2, 3, 2)), (8, (2, 2, 1, 3))):
        n = int(np.prod(grid))
        np.testing.assert_array_equal(dirs.seq_to_tok_table(K, n, grid).numpy(), f[f"K{K}"])
