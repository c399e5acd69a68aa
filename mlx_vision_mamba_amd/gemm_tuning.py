"""GEMM selections for the VisionMamba projections on MI355X.

The block's projections (in_proj, x_proj, dt_proj, out_proj and their
gradients) are plain fp32 GEMMs on the ROCm BLAS libraries.  PyTorch's
TunableOp can pick, per GEMM shape, the fastest of the rocBLAS and
hipBLASLt solutions; ``tuning/gemm_mi355x_visionmamba2d.csv`` holds the
picks measured on MI355X for the VisionMamba-2D training step (batch 32,
224x224x1, patch 16, E = 384, K = 4).  ``load()`` turns TunableOp on in
read-only mode with that file: listed shapes use the recorded solution,
other shapes keep the library default, and nothing is tuned at run time.
The file's validator lines (PyTorch, HIP, hipBLASLt, rocBLAS versions,
gfx arch) must match the running stack, or TunableOp ignores its entries.
"""

from __future__ import annotations

import os

import torch

DEFAULT_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tuning",
                            "gemm_mi355x_visionmamba2d.csv")


def load(path: str = DEFAULT_FILE) -> bool:
    """Use the recorded GEMM solutions of ``path``; False if it is missing."""
    if not os.path.exists(path):
        return False
    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(False)
    torch.cuda.tunable.record_untuned_enable(False)
    torch.cuda.tunable.set_filename(path, insert_device_ordinal=False)
    return bool(torch.cuda.tunable.read_file(path))


def start_tuning(path: str) -> None:
    """Tune every GEMM the process runs from now on; the picks are written to
    ``path`` when the process exits."""
    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(True)
    torch.cuda.tunable.set_max_tuning_duration(50)
    torch.cuda.tunable.set_max_tuning_iterations(50)
    torch.cuda.tunable.set_filename(path, insert_device_ordinal=False)
