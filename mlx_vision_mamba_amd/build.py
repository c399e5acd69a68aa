"""Builds libmvm_scan.so (the HIP kernels + C ABI) in-tree for gfx950.

    python -m mlx_vision_mamba_amd.build

Every HIP source is compiled with hipcc for gfx950 only, with packed-FP32
VALU forms disabled (-Xclang -target-feature -Xclang -packed-fp32-ops), and
linked into one shared library next to this file.  The library links the
HIP runtime by soname (libamdhip64.so.7); it must be loaded after
``import torch`` so that it binds to the runtime torch already loaded.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(PKG, "libmvm_scan.so")
SOURCES = ["capi.hip", "scan_fwd.hip", "scan_bwd.hip", "conv.hip", "layernorm.hip", "optim.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def cflags():
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-result",
        f"-I{INCLUDE}", f"-I{CSRC}",
    ]


def _compile(src: str, obj: str, extra):
    cmd = [hipcc(), *cflags(), *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    # hipcc's host pass does not know the packed-fp32 feature; drop that noise
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in res.stderr.splitlines() if noise not in ln and ln.strip()]
    return "\n".join(msgs)


def build(verbose: bool = False, extra=()) -> str:
    """Compile every HIP source and link LIB; returns its path."""
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        futs = [ex.submit(_compile, s, o, list(extra)) for s, o in zip(SOURCES, objs)]
        for f in futs:
            msg = f.result()
            if verbose and msg:
                print(msg, file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
