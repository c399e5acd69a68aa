"""ctypes binding of the float64 C oracle (oracle/scan_ref.c).

TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle_scan.so")
_lib = None


def build():
    """Compile scan_ref.c with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        lib = ctypes.CDLL(_SO)
        i64, fp, dp = ctypes.c_int64, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_double)
        lib.oracle_scan_fwd.argtypes = [i64] * 4 + [fp] * 6 + [dp]
        lib.oracle_scan_fwd.restype = ctypes.c_int
        lib.oracle_scan_vjp.argtypes = [i64] * 4 + [fp] * 7 + [dp] * 6
        lib.oracle_scan_vjp.restype = ctypes.c_int
        lib.oracle_ddelta_scale.argtypes = [i64] * 4 + [fp] * 6 + [dp]
        lib.oracle_ddelta_scale.restype = ctypes.c_int
        lib.oracle_dA_scale.argtypes = [i64] * 4 + [fp] * 6 + [dp]
        lib.oracle_dA_scale.restype = ctypes.c_int
        lib.oracle_scan_fwd_f64.argtypes = [i64] * 4 + [dp] * 7
        lib.oracle_scan_fwd_f64.restype = ctypes.c_int
        lib.oracle_scan_vjp_f64.argtypes = [i64] * 4 + [dp] * 13
        lib.oracle_scan_vjp_f64.restype = ctypes.c_int
        lib.oracle_scan_all.argtypes = [i64] * 4 + [fp] * 7 + [dp] * 8
        lib.oracle_scan_all.restype = ctypes.c_int
        lib.oracle_scan_mag_fwd.argtypes = [i64] * 4 + [dp] * 13
        lib.oracle_scan_mag_fwd.restype = ctypes.c_int
        lib.oracle_scan_mag_vjp.argtypes = [i64] * 4 + [dp] * 20
        lib.oracle_scan_mag_vjp.restype = ctypes.c_int
        lib.oracle_num_threads.restype = ctypes.c_int
        _lib = lib
    return _lib


def _f32(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _f64(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float64))


def _p(a, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def num_threads() -> int:
    return int(_load().oracle_num_threads())


def scan_fwd(u, delta, A, B, C, D):
    """float64 y for float32 inputs (B,L,D),(B,L,D),(D,N),(B,L,N),(B,L,N),(D,)."""
    lib = _load()
    u, delta, A, B, C, D = map(_f32, (u, delta, A, B, C, D))
    bsz, L, d = u.shape
    n = A.shape[1]
    y = np.empty((bsz, L, d), dtype=np.float64)
    fp = ctypes.c_float
    rc = lib.oracle_scan_fwd(bsz, L, d, n, _p(u, fp), _p(delta, fp), _p(A, fp),
                             _p(B, fp), _p(C, fp), _p(D, fp), _p(y, ctypes.c_double))
    if rc != 0:
        raise RuntimeError(f"oracle_scan_fwd failed ({rc})")
    return y


def scan_vjp(u, delta, A, B, C, D, g):
    """float64 (du, ddelta, dA, dB, dC, dD)."""
    lib = _load()
    u, delta, A, B, C, D, g = map(_f32, (u, delta, A, B, C, D, g))
    bsz, L, d = u.shape
    n = A.shape[1]
    outs = [np.empty((bsz, L, d)), np.empty((bsz, L, d)), np.empty((d, n)),
            np.empty((bsz, L, n)), np.empty((bsz, L, n)), np.empty((d,))]
    fp, dp = ctypes.c_float, ctypes.c_double
    rc = lib.oracle_scan_vjp(bsz, L, d, n, _p(u, fp), _p(delta, fp), _p(A, fp),
                             _p(B, fp), _p(C, fp), _p(D, fp), _p(g, fp),
                             *[_p(o, dp) for o in outs])
    if rc != 0:
        raise RuntimeError(f"oracle_scan_vjp failed ({rc})")
    return tuple(outs)


def ddelta_scale(u, delta, A, B, C, g):
    """float64 S[b,t,d] = sum_n |lam_n| (|A_n e_n h_{t-1,n}| + |B_n u_t|):
    the cancellation scale of ddelta (see scan_ref.c)."""
    lib = _load()
    u, delta, A, B, C, g = map(_f32, (u, delta, A, B, C, g))
    bsz, L, d = u.shape
    n = A.shape[1]
    out = np.empty((bsz, L, d), dtype=np.float64)
    fp = ctypes.c_float
    rc = lib.oracle_ddelta_scale(bsz, L, d, n, _p(u, fp), _p(delta, fp), _p(A, fp), _p(B, fp),
                                 _p(C, fp), _p(g, fp), _p(out, ctypes.c_double))
    if rc != 0:
        raise RuntimeError(f"oracle_ddelta_scale failed ({rc})")
    return out


def dA_scale(u, delta, A, B, C, g):
    """float64 S[d,n] = sum_{b,t} |lam_t delta_t e_t h_{t-1}|: the
    cancellation scale of dA (see scan_ref.c)."""
    lib = _load()
    u, delta, A, B, C, g = map(_f32, (u, delta, A, B, C, g))
    bsz, L, d = u.shape
    n = A.shape[1]
    out = np.empty((d, n), dtype=np.float64)
    fp = ctypes.c_float
    rc = lib.oracle_dA_scale(bsz, L, d, n, _p(u, fp), _p(delta, fp), _p(A, fp), _p(B, fp),
                             _p(C, fp), _p(g, fp), _p(out, ctypes.c_double))
    if rc != 0:
        raise RuntimeError(f"oracle_dA_scale failed ({rc})")
    return out


def scan_fwd_f64(u, delta, A, B, C, D):
    """``scan_fwd`` for float64 inputs (the float64 module restatements)."""
    lib = _load()
    u, delta, A, B, C, D = map(_f64, (u, delta, A, B, C, D))
    bsz, L, d = u.shape
    n = A.shape[1]
    y = np.empty((bsz, L, d), dtype=np.float64)
    dp = ctypes.c_double
    rc = lib.oracle_scan_fwd_f64(bsz, L, d, n, *[_p(a, dp) for a in (u, delta, A, B, C, D, y)])
    if rc != 0:
        raise RuntimeError(f"oracle_scan_fwd_f64 failed ({rc})")
    return y


def scan_vjp_f64(u, delta, A, B, C, D, g):
    """``scan_vjp`` for float64 inputs."""
    lib = _load()
    u, delta, A, B, C, D, g = map(_f64, (u, delta, A, B, C, D, g))
    bsz, L, d = u.shape
    n = A.shape[1]
    outs = [np.empty((bsz, L, d)), np.empty((bsz, L, d)), np.empty((d, n)),
            np.empty((bsz, L, n)), np.empty((bsz, L, n)), np.empty((d,))]
    dp = ctypes.c_double
    rc = lib.oracle_scan_vjp_f64(bsz, L, d, n, *[_p(a, dp) for a in (u, delta, A, B, C, D, g)],
                                 *[_p(o, dp) for o in outs])
    if rc != 0:
        raise RuntimeError(f"oracle_scan_vjp_f64 failed ({rc})")
    return tuple(outs)


def scan_all(u, delta, A, B, C, D, g):
    """(y, (du, ddelta, dA, dB, dC, dD), S) in one pass: the results of
    ``scan_fwd``, ``scan_vjp`` and ``ddelta_scale`` on the same inputs."""
    lib = _load()
    u, delta, A, B, C, D, g = map(_f32, (u, delta, A, B, C, D, g))
    bsz, L, d = u.shape
    n = A.shape[1]
    outs = [np.empty((bsz, L, d)), np.empty((bsz, L, d)), np.empty((bsz, L, d)), np.empty((d, n)),
            np.empty((bsz, L, n)), np.empty((bsz, L, n)), np.empty((d,)), np.empty((bsz, L, d))]
    fp, dp = ctypes.c_float, ctypes.c_double
    rc = lib.oracle_scan_all(bsz, L, d, n, *[_p(a, fp) for a in (u, delta, A, B, C, D, g)],
                             *[_p(o, dp) for o in outs])
    if rc != 0:
        raise RuntimeError(f"oracle_scan_all failed ({rc})")
    return outs[0], tuple(outs[1:7]), outs[7]


def scan_mag_fwd(values, mags):
    """Error-magnitude companion of the scan forward (scan_ref.c
    oracle_scan_mag_fwd).  values = (u, delta, A, B, C, D), mags = (Mu, Md,
    MA, MB, MC, MD), float64 with the shapes of the scan's inputs; returns
    My (B, L, D)."""
    lib = _load()
    vals = list(map(_f64, values))
    ms = list(map(_f64, mags))
    bsz, L, d = vals[0].shape
    n = vals[2].shape[1]
    for v, m in zip(vals, ms):
        if v.shape != m.shape:
            raise ValueError(f"magnitude shape {m.shape} != value shape {v.shape}")
    out = np.empty((bsz, L, d))
    dp = ctypes.c_double
    rc = lib.oracle_scan_mag_fwd(bsz, L, d, n, *[_p(a, dp) for a in vals + ms], _p(out, dp))
    if rc != 0:
        raise RuntimeError(f"oracle_scan_mag_fwd failed ({rc})")
    return out


def scan_mag_vjp(values, mags, g, Mg):
    """Error magnitudes of the scan's six gradients (du, ddelta, dA, dB, dC,
    dD) for the actual cotangent g of y and its magnitude Mg (scan_ref.c
    oracle_scan_mag_vjp)."""
    lib = _load()
    vals = list(map(_f64, values))
    ms = list(map(_f64, mags))
    g, Mg = _f64(g), _f64(Mg)
    bsz, L, d = vals[0].shape
    n = vals[2].shape[1]
    outs = [np.empty((bsz, L, d)), np.empty((bsz, L, d)), np.empty((d, n)),
            np.empty((bsz, L, n)), np.empty((bsz, L, n)), np.empty((d,))]
    dp = ctypes.c_double
    rc = lib.oracle_scan_mag_vjp(bsz, L, d, n, *[_p(a, dp) for a in vals + ms + [g, Mg]],
                                 *[_p(o, dp) for o in outs])
    if rc != 0:
        raise RuntimeError(f"oracle_scan_mag_vjp failed ({rc})")
    return tuple(outs)
