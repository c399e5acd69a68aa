"""Host-side checks of the benchmark's contract (no GPU): the algorithmic
byte counts the roofline divides by, the counter figures it reads from the
committed profile, and the single-GPU guard."""

import os
import subprocess
import sys

import bench
from mlx_vision_mamba_amd import scan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_algorithmic_bytes_of_the_measured_calls():
    # plain scan, B=2 L=196 D=1536 N=16 fp32: every tensor read / written once
    fwd, vjp = scan.algorithmic_bytes(2, 196, 1536, 16, 4, 4)
    assert fwd + vjp == 19_731_456
    # B=8 L=16384 D=1536 N=16, bf16 u/B/C/y/grads, fp32 delta / A / D
    fwd, vjp = scan.algorithmic_bytes(8, 16384, 1536, 16, 2, 2)
    assert fwd + vjp == 4_454_664_192
    # the fused call of one VisionMamba-2D layer: B*K = 128 rows, L=196, D=768
    fwd, vjp = scan.algorithmic_bytes_fused(128, 196, 768, 16, 4)
    assert (fwd, vjp) == (388_784_128, 623_427_584)
    # by hand: the VJP reads u, delta_raw, dy, z, y_raw and writes du,
    # ddelta_raw, dz (8 per-(b,t,d) fp32 tensors), reads B, C and writes
    # dB, dC (4 per-(b,t,n)), reads A, D, bias and writes dA, dD, dbias
    BLD, BLN = 128 * 196 * 768, 128 * 196 * 16
    assert vjp == 4 * (8 * BLD + 4 * BLN) + 4 * (768 * 16 * 8 + 768 * 8 + 768 * 8)


def test_secondary_flop_rate():
    # 37 flop per element (forward + VJP of the reference formula): 1e9
    # elements in 1 ms is 37 TFLOP/s, 23.5 % of the 157.3 TFLOP/s fp32 peak
    sec = bench.secondary_flops(1_000_000_000, 1e-3)
    assert sec["achieved_TFLOPs"] == 37.0
    assert abs(sec["frac"] - 37.0 / 157.3) < 1e-4
    assert sec["flop_per_element"] == 37 and sec["exp_per_element"] == 3
    # the VisionMamba step's fused calls: B*K = 128 scans of 196 x 768 x 16
    assert 32 * 4 * 196 * 768 * 16 == 308_281_344


def test_profile_figures_read_by_the_bench():
    traffic = bench.measured_traffic("bwd_call_hbm_bytes")
    assert isinstance(traffic, int)
    # measured HBM bytes cover at least the algorithmic bytes of the call
    assert traffic >= 623_427_584
    busy = bench.measured_traffic("bwd_valu_busy_per_simd", float)
    assert 0.0 < busy <= 1.0
    assert bench.measured_traffic("no_such_key") is None


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr and res.stdout == ""
