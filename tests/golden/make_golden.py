"""Writes the golden fixtures of this directory from the float64 oracle.

    python tests/golden/make_golden.py

The reference has no tests, golden vectors or fixtures of its own, and MLX
cannot run here, so the expected outputs come from the oracle (oracle/),
after tests/test_oracle.py and tests/test_oracle_blocks.py have pinned it
by closed forms, library routines, autograd and finite differences.  Each
fixture holds seeded float32 inputs and the float64 expected outputs:

  scan_small.npz    plain scan, B=2 L=37 D=48 N=16 (random decays):
                    y, du, ddelta, dA, dB, dC, dD and the ddelta
                    cancellation scale S (mamba_block.py:20-74,
                    mamba_metal_fused.py:66-145, :213-224)
  fused_small.npz   the block's prologue / epilogue around the scan,
                    B=2 L=23 D=40 N=8 with dt bias and gate
                    (mamba_block.py:180-190), and S_raw, the
                    cancellation scale of the delta_raw gradient
  directions.npz    scan-order tables of K=4 (3,4), K=6 (2,3,2),
                    K=8 (2,2,1,3) grids (mamba_block.py:407-533)

tests/test_golden.py checks that the oracle still reproduces them and that
the direction tables of the product equal them; tests/test_gpu_golden.py
checks the HIP path against them.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import ref_lib, scan_oracle as so  # noqa: E402


def scan_case():
    rng = np.random.default_rng(40)
    bsz, L, D, N = 2, 37, 48, 16
    u = rng.standard_normal((bsz, L, D))
    delta = np.logaddexp(0.0, rng.standard_normal((bsz, L, D)) * 0.5 - 3.0)
    A = -np.exp(rng.standard_normal((D, N)) * 0.5)
    Bm = rng.standard_normal((bsz, L, N))
    Cm = rng.standard_normal((bsz, L, N))
    Dv = rng.standard_normal(D)
    g = rng.standard_normal((bsz, L, D))
    ins = [a.astype(np.float32) for a in (u, delta, A, Bm, Cm, Dv, g)]
    y = ref_lib.scan_fwd(*ins[:6])
    du, ddelta, dA, dB, dC, dD = ref_lib.scan_vjp(*ins)
    S = ref_lib.ddelta_scale(*ins[:5], ins[6])
    names = ("u", "delta", "A", "B", "C", "D", "g")
    return dict(zip(names, ins), y=y, du=du, ddelta=ddelta, dA=dA, dB=dB, dC=dC, dD=dD, S=S)


def fused_case():
    rng = np.random.default_rng(41)
    bsz, L, D, N = 2, 23, 40, 8
    u = rng.standard_normal((bsz, L, D))
    draw = rng.standard_normal((bsz, L, D)) * 1.5 - 3.0
    draw[0, 0, :3] = 22.0                    # softplus's linear branch
    bias = rng.standard_normal(D) * 0.5
    A = -np.exp(rng.standard_normal((D, N)) * 0.5)
    Bm = rng.standard_normal((bsz, L, N))
    Cm = rng.standard_normal((bsz, L, N))
    Dv = rng.standard_normal(D)
    z = rng.standard_normal((bsz, L, D)) * 2.0
    g = rng.standard_normal((bsz, L, D))
    ins = [a.astype(np.float32) for a in (u, draw, bias, A, Bm, Cm, Dv, z, g)]
    f64 = [a.astype(np.float64) for a in ins]
    y, y_raw, _ = so.fused_fwd(*f64[:8])
    du, ddr, db, dA, dB, dC, dD, dz = so.fused_vjp(*f64)
    # cancellation scale of ddelta_raw = ddelta * sigmoid(x): the scan's S for
    # delta = softplus(x) and upstream g * silu(z), times sigmoid(x)
    x = f64[1] + f64[2]
    _, _, delta = so.fused_fwd(*f64[:8])
    gs = f64[8] * f64[7] * so.sigmoid(f64[7])
    S_raw = ref_lib.ddelta_scale(ins[0], delta, ins[3], ins[4], ins[5], gs) * so.sigmoid(x)
    names = ("u", "delta_raw", "bias", "A", "B", "C", "D", "z", "g")
    return dict(zip(names, ins), y=y, y_raw=y_raw, du=du, ddelta_raw=ddr, dbias=db, dA=dA,
                dB=dB, dC=dC, dD=dD, dz=dz, S_raw=S_raw)


def direction_tables():
    out = {}
    for K, grid in ((4, (3, 4)), (6, (2, 3, 2)), (8, (2, 2, 1, 3))):
        n = int(np.prod(grid))
        out[f"K{K}"] = np.stack([so.seq_to_token(n, grid, *so.direction_axis_order(K, k))
                                 for k in range(K)]).astype(np.int32)
    return out


def main():
    np.savez_compressed(os.path.join(HERE, "scan_small.npz"), **scan_case())
    np.savez_compressed(os.path.join(HERE, "fused_small.npz"), **fused_case())
    np.savez_compressed(os.path.join(HERE, "directions.npz"), **direction_tables())


if __name__ == "__main__":
    main()
