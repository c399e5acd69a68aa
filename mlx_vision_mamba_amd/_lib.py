"""ctypes binding of libmvm_scan.so (the C ABI declared in include/mvm_scan.h).

The library is loaded after ``import torch`` so that its HIP runtime
dependency (soname libamdhip64.so.7) resolves to the runtime torch already
loaded: device pointers and hipStream_t handles from torch are then valid in
the library.  A missing library raises ImportError -- there is no fallback.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded before the HIP library)

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libmvm_scan.so")

MVM_OK = 0
MVM_ERR_INVALID_ARG = -1
MVM_ERR_UNSUPPORTED = -2
MVM_ERR_WORKSPACE = -3
MVM_ERR_HIP = -4
MVM_F32 = 0
MVM_BF16 = 1
MVM_MAX_DSTATE = 16
ABI_VERSION = 4
MVM_NORM_MAX_COLS = 1024

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_vp = ctypes.c_void_p


class ScanDesc(ctypes.Structure):
    """Mirror of ``mvm_scan_desc`` (include/mvm_scan.h)."""

    _fields_ = [
        ("batch", _i64), ("seqlen", _i64), ("dim", _i64), ("dstate", _i64), ("ndir", _i64),
        ("x_stride_b", _i64), ("x_stride_k", _i64), ("x_stride_t", _i64),
        ("bc_stride_b", _i64), ("bc_stride_k", _i64), ("bc_stride_t", _i64),
        ("seq_to_tok", _vp),
        ("in_dtype", _i32), ("out_dtype", _i32), ("chunk_len", _i32), ("reserved", _i32),
    ]


class FusedDesc(ctypes.Structure):
    """Mirror of ``mvm_scan_fused_desc`` (include/mvm_scan.h)."""

    _fields_ = [
        ("scan", ScanDesc),
        ("dt_stride_b", _i64), ("dt_stride_k", _i64), ("dt_stride_t", _i64),
        ("y_stride_b", _i64), ("y_stride_k", _i64), ("y_stride_t", _i64),
        ("z_stride_b", _i64), ("z_stride_k", _i64), ("z_stride_t", _i64),
        ("a_is_log", _i32), ("reserved", _i32),
    ]


class ConvDesc(ctypes.Structure):
    """Mirror of ``mvm_conv_desc`` (include/mvm_conv.h)."""

    _fields_ = [
        ("batch", _i64), ("seqlen", _i64), ("dim", _i64), ("ndir", _i64), ("kwidth", _i64),
        ("x_stride_b", _i64), ("x_stride_k", _i64), ("x_stride_t", _i64),
        ("y_stride_b", _i64), ("y_stride_k", _i64), ("y_stride_t", _i64),
        ("seq_to_tok", _vp),
        ("dx_stride_b", _i64), ("dx_stride_k", _i64), ("dx_stride_t", _i64),
    ]


class NormDesc(ctypes.Structure):
    """Mirror of ``mvm_norm_desc`` (include/mvm_norm.h)."""

    _fields_ = [
        ("rows", _i64), ("cols", _i64), ("x_stride", _i64), ("y_stride", _i64),
        ("eps", ctypes.c_float), ("reserved", _i32),
    ]


class AdamwTensor(ctypes.Structure):
    """Mirror of ``mvm_adamw_tensor`` (include/mvm_optim.h)."""

    _fields_ = [("param", _vp), ("grad", _vp), ("numel", _i64), ("state_offset", _i64)]


class AdamwHparams(ctypes.Structure):
    """Mirror of ``mvm_adamw_hparams`` (include/mvm_optim.h)."""

    _fields_ = [
        ("lr", ctypes.c_float), ("beta1", ctypes.c_float), ("beta2", ctypes.c_float),
        ("eps", ctypes.c_float), ("weight_decay", ctypes.c_float), ("reserved", _i32),
    ]


# symbol -> (restype, argtypes); every entry point of include/mvm_scan.h,
# include/mvm_conv.h, include/mvm_norm.h, include/mvm_optim.h and the test
# hook of include/mvm_testing.h
SIGNATURES = {
    "mvm_abi_version": (ctypes.c_int, []),
    "mvm_last_error": (ctypes.c_char_p, []),
    "mvm_scan_validate": (ctypes.c_int, [ctypes.POINTER(ScanDesc)]),
    "mvm_scan_ckpt_elems": (_i64, [ctypes.POINTER(ScanDesc)]),
    "mvm_scan_workspace_bytes": (_i64, [ctypes.POINTER(ScanDesc), ctypes.c_int]),
    "mvm_scan_chunk_len": (_i64, [ctypes.POINTER(ScanDesc)]),
    "mvm_scan_fwd": (ctypes.c_int, [ctypes.POINTER(ScanDesc)] + [_vp] * 9 + [ctypes.c_size_t, _vp]),
    "mvm_scan_bwd": (ctypes.c_int, [ctypes.POINTER(ScanDesc)] + [_vp] * 15 + [ctypes.c_size_t, _vp]),
    "mvm_scan_noalloc_scratch_bytes": (_i64, []),
    "mvm_scan_bwd_noalloc": (ctypes.c_int, [ctypes.POINTER(ScanDesc)] + [_vp] * 15),
    "mvm_scan_fused_validate": (ctypes.c_int, [ctypes.POINTER(FusedDesc)]),
    "mvm_scan_fused_workspace_bytes": (_i64, [ctypes.POINTER(FusedDesc), ctypes.c_int, ctypes.c_int]),
    "mvm_scan_fused_fwd": (ctypes.c_int, [ctypes.POINTER(FusedDesc)] + [_vp] * 12 + [ctypes.c_size_t, _vp]),
    "mvm_scan_fused_bwd": (ctypes.c_int, [ctypes.POINTER(FusedDesc)] + [_vp] * 20 + [ctypes.c_size_t, _vp]),
    "mvm_conv_validate": (ctypes.c_int, [ctypes.POINTER(ConvDesc)]),
    "mvm_conv_workspace_bytes": (_i64, [ctypes.POINTER(ConvDesc)]),
    "mvm_conv_silu_fwd": (ctypes.c_int, [ctypes.POINTER(ConvDesc)] + [_vp] * 5),
    "mvm_conv_silu_bwd": (ctypes.c_int, [ctypes.POINTER(ConvDesc)] + [_vp] * 8 + [ctypes.c_size_t, _vp]),
    "mvm_norm_validate": (ctypes.c_int, [ctypes.POINTER(NormDesc)]),
    "mvm_norm_workspace_bytes": (_i64, [ctypes.POINTER(NormDesc)]),
    "mvm_layernorm_fwd": (ctypes.c_int, [ctypes.POINTER(NormDesc)] + [_vp] * 7),
    "mvm_layernorm_bwd": (ctypes.c_int, [ctypes.POINTER(NormDesc)] + [_vp] * 10 + [ctypes.c_size_t, _vp]),
    "mvm_adamw_step": (ctypes.c_int, [ctypes.POINTER(AdamwTensor), _i32, ctypes.POINTER(AdamwHparams),
                                      _vp, _vp, _vp, _vp]),
    "mvm_selftest_lanes": (ctypes.c_int, [_vp, _vp]),
}

_lib = None


class ScanError(RuntimeError):
    """A negative status from libmvm_scan; ``code`` holds the MVM_ERR_* value."""

    def __init__(self, code, msg):
        super().__init__(f"libmvm_scan error {code}: {msg}")
        self.code = code


def lib():
    """The loaded library (ImportError if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m mlx_vision_mamba_amd.build` "
                "(the HIP extension is required; there is no CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        ver = handle.mvm_abi_version()
        if ver != ABI_VERSION:
            raise ImportError(f"libmvm_scan ABI {ver} != expected {ABI_VERSION}")
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().mvm_last_error().decode()


def check(rc: int) -> int:
    if rc < 0:
        raise ScanError(rc, last_error())
    return rc
