"""Host-side checks of the C ABI (no GPU needed, no kernel launches).

The library must load on a machine without a GPU, export every entry point
its headers declare, and reject bad arguments on the host -- before anything
is enqueued -- with the documented error codes.
"""

import ctypes
import os
import re

import pytest
import torch

from mlx_vision_mamba_amd import _lib, scan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = []
    for hdr in ("mvm_scan.h", "mvm_conv.h", "mvm_norm.h", "mvm_optim.h", "mvm_testing.h"):
        text = open(os.path.join(ROOT, "include", hdr)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(mvm_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _declared_functions()
    assert "mvm_scan_fwd" in declared and "mvm_scan_bwd" in declared
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.SIGNATURES)
    assert lib.mvm_abi_version() == _lib.ABI_VERSION


def _header_arity():
    """Parameter count of every function declared in the headers."""
    out = {}
    for hdr in ("mvm_scan.h", "mvm_conv.h", "mvm_norm.h", "mvm_optim.h", "mvm_testing.h"):
        text = open(os.path.join(ROOT, "include", hdr)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for name, params in re.findall(r"\b(mvm_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
            params = params.strip()
            out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_seqlen_limit_leaves_room_for_tile_rows():
    """Kernel positions are int32 and a tile's rows are formed as position +
    up to 63 before they are clamped, so seqlen is capped at 2^31 - 65; the
    last chunk's end is formed in 64 bits, so a chunk_len that reaches past
    2^31 - 1 is accepted."""
    limit = 2 ** 31 - 65
    d = _desc(B=1, L=limit, D=1, N=1)
    d.x_stride_b, d.x_stride_t, d.bc_stride_b, d.bc_stride_t = limit, 1, limit, 1
    d.chunk_len = 2 ** 30
    assert _validate(d) == 0
    d.seqlen = limit + 1
    d.x_stride_b = d.bc_stride_b = limit + 1
    assert _validate(d) == _lib.MVM_ERR_UNSUPPORTED
    assert b"seqlen" in _lib.lib().mvm_last_error()


def test_ctypes_signatures_match_header_arity():
    arity = _header_arity()
    assert set(arity) == set(_lib.SIGNATURES)
    for name, (_, args) in _lib.SIGNATURES.items():
        assert len(args) == arity[name], name


def _desc(B=2, L=40, D=24, N=16, K=1):
    d = _lib.ScanDesc()
    d.batch, d.seqlen, d.dim, d.dstate, d.ndir = B, L, D, N, K
    d.x_stride_b, d.x_stride_t, d.x_stride_k = L * K * D, K * D, D
    d.bc_stride_b, d.bc_stride_t, d.bc_stride_k = L * K * N, K * N, N
    return d


def _validate(d):
    return _lib.lib().mvm_scan_validate(ctypes.byref(d))


def test_valid_desc_and_sizes():
    d = _desc()
    assert _validate(d) == 0
    lib = _lib.lib()
    assert lib.mvm_scan_ckpt_elems(ctypes.byref(d)) == 2 * 1 * 5 * 24 * 16   # ceil(40/8)=5
    assert lib.mvm_scan_chunk_len(ctypes.byref(d)) % 16 == 0
    for which in (0, 1, 2):
        assert lib.mvm_scan_workspace_bytes(ctypes.byref(d), which) >= 0
    assert lib.mvm_scan_workspace_bytes(ctypes.byref(d), 7) == _lib.MVM_ERR_INVALID_ARG


@pytest.mark.parametrize("field,value,code", [
    ("dstate", 17, _lib.MVM_ERR_UNSUPPORTED),      # the reference's float h[16] cap
    ("dstate", 0, _lib.MVM_ERR_UNSUPPORTED),
    ("batch", -1, _lib.MVM_ERR_INVALID_ARG),
    ("seqlen", -3, _lib.MVM_ERR_INVALID_ARG),
    ("ndir", 0, _lib.MVM_ERR_INVALID_ARG),
    ("in_dtype", 7, _lib.MVM_ERR_UNSUPPORTED),
    ("out_dtype", 2, _lib.MVM_ERR_UNSUPPORTED),
    ("chunk_len", 24, _lib.MVM_ERR_INVALID_ARG),
    ("x_stride_t", 3, _lib.MVM_ERR_INVALID_ARG),
    ("bc_stride_t", 2, _lib.MVM_ERR_INVALID_ARG),
    ("x_stride_b", -5, _lib.MVM_ERR_INVALID_ARG),
    ("x_stride_b", 0, _lib.MVM_ERR_INVALID_ARG),    # batch 2 broadcast: du would race
    ("bc_stride_b", 0, _lib.MVM_ERR_INVALID_ARG),
    ("x_stride_b", 24 * 39, _lib.MVM_ERR_INVALID_ARG),  # batch 1 overlaps batch 0's last row
])
def test_bad_descriptors_rejected(field, value, code):
    d = _desc()
    setattr(d, field, value)
    assert _validate(d) == code
    assert _lib.last_error() != ""


@pytest.mark.parametrize("field", ["x_stride_k", "bc_stride_k"])
def test_direction_stride_zero_rejected_with_several_directions(field):
    d = _desc(K=2)
    assert _validate(d) == 0
    setattr(d, field, 0)
    assert _validate(d) == _lib.MVM_ERR_INVALID_ARG
    assert "overlap" in _lib.last_error()


def test_size_one_dimensions_take_any_stride():
    """A dimension of size 1 is never stepped, so its stride is free."""
    d = _desc(B=1, K=1)
    d.x_stride_b = d.bc_stride_b = 0
    d.x_stride_k = d.bc_stride_k = 0
    assert _validate(d) == 0
    # interleaved layouts that do not overlap pass: (b, t) strides (24, 48)
    d = _desc(B=2, L=40, D=24)
    d.x_stride_b, d.x_stride_t = 24, 48
    assert _validate(d) == 0


def test_null_pointers_rejected_before_launch():
    lib = _lib.lib()
    d = _desc()
    null = ctypes.c_void_p(0)
    rc = lib.mvm_scan_fwd(ctypes.byref(d), *([null] * 9), 0, null)
    assert rc == _lib.MVM_ERR_INVALID_ARG
    assert "NULL" in _lib.last_error()
    rc = lib.mvm_scan_bwd(ctypes.byref(d), *([null] * 15), 0, null)
    assert rc == _lib.MVM_ERR_INVALID_ARG


def test_small_workspace_rejected_before_launch():
    lib = _lib.lib()
    d = _desc(L=4096, D=64)
    need = lib.mvm_scan_workspace_bytes(ctypes.byref(d), 1)
    assert need > 0
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: validation fails first
    rc = lib.mvm_scan_bwd(ctypes.byref(d), *([fake] * 15), need - 1, ctypes.c_void_p(0))
    assert rc == _lib.MVM_ERR_WORKSPACE
    assert "workspace" in _lib.last_error()


@pytest.mark.parametrize("B,L,D", [(0, 40, 24), (2, 0, 24), (2, 40, 0)])
def test_empty_forward_is_a_no_op(B, L, D):
    """An empty (b, t, d) range needs no buffers: the forward validates and
    returns before any launch, with NULL tensor pointers and no workspace."""
    lib = _lib.lib()
    d = _desc(B=B, L=L, D=D)
    assert lib.mvm_scan_validate(ctypes.byref(d)) == _lib.MVM_OK
    assert lib.mvm_scan_ckpt_elems(ctypes.byref(d)) == 0
    assert lib.mvm_scan_workspace_bytes(ctypes.byref(d), 0) == 0
    assert lib.mvm_scan_workspace_bytes(ctypes.byref(d), 1) >= 0
    null = ctypes.c_void_p(0)
    assert lib.mvm_scan_fwd(ctypes.byref(d), *([null] * 9), 0, null) == _lib.MVM_OK
    # the backward still owes dA and dD (zero sums over the empty range)
    if D > 0:
        assert lib.mvm_scan_bwd(ctypes.byref(d), *([null] * 15), 0, null) == _lib.MVM_ERR_INVALID_ARG
        assert "dA" in _lib.last_error()


def test_null_desc():
    assert _lib.lib().mvm_scan_validate(None) == _lib.MVM_ERR_INVALID_ARG


def test_auto_chunking_fills_the_chip_for_long_sequences():
    lib = _lib.lib()
    d = _desc(B=8, L=16384, D=1536)
    cl = lib.mvm_scan_chunk_len(ctypes.byref(d))
    nchunk = -(-16384 // cl)
    waves = 8 * 24 * 4 * nchunk
    assert cl % 16 == 0 and waves >= 16384 and 256 <= cl <= 1024
    d2 = _desc(B=32, L=196, D=768, K=4)
    assert lib.mvm_scan_chunk_len(ctypes.byref(d2)) >= 196   # enough rows: one chunk


def test_cpu_tensors_raise_no_fallback():
    x = torch.randn(1, 8, 4)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        scan.selective_scan(x, x.abs(), -torch.ones(4, 16), torch.randn(1, 8, 16),
                            torch.randn(1, 8, 16), torch.ones(4))


def test_scan_mode_registry():
    for m in scan.SCAN_MODES:
        assert callable(scan.get_scan_fn(m))
    with pytest.raises(ValueError, match="unknown scan_mode"):
        scan.get_scan_fn("metal_fast")


def test_shape_errors():
    with pytest.raises(ValueError):
        scan.scan_forward(torch.zeros(1, 2, 1, 3), torch.zeros(1, 2, 1, 3), torch.zeros(1, 3, 17),
                          torch.zeros(1, 2, 1, 17), torch.zeros(1, 2, 1, 17), torch.zeros(1, 3))


def _cdesc(B=2, L=20, D=24, K=1, kc=4):
    d = _lib.ConvDesc()
    d.batch, d.seqlen, d.dim, d.ndir, d.kwidth = B, L, D, K, kc
    d.x_stride_b, d.x_stride_t, d.x_stride_k = L * K * 2 * D, K * 2 * D, 2 * D
    d.y_stride_b, d.y_stride_t, d.y_stride_k = L * K * D, K * D, D
    d.dx_stride_b, d.dx_stride_t, d.dx_stride_k = L * K * D, K * D, D
    return d


@pytest.mark.parametrize("field,value,code", [
    ("kwidth", 9, _lib.MVM_ERR_UNSUPPORTED), ("kwidth", 0, _lib.MVM_ERR_UNSUPPORTED),
    ("ndir", 0, _lib.MVM_ERR_INVALID_ARG), ("batch", -2, _lib.MVM_ERR_INVALID_ARG),
    ("y_stride_t", 3, _lib.MVM_ERR_INVALID_ARG), ("x_stride_k", -1, _lib.MVM_ERR_INVALID_ARG),
    ("dx_stride_t", 3, _lib.MVM_ERR_INVALID_ARG), ("dx_stride_b", -1, _lib.MVM_ERR_INVALID_ARG),
])
def test_conv_bad_descriptors_rejected(field, value, code):
    lib = _lib.lib()
    d = _cdesc()
    assert lib.mvm_conv_validate(ctypes.byref(d)) == 0
    assert lib.mvm_conv_workspace_bytes(ctypes.byref(d)) > 0
    setattr(d, field, value)
    assert lib.mvm_conv_validate(ctypes.byref(d)) == code


def test_conv_null_and_workspace_rejected_before_launch():
    lib = _lib.lib()
    d = _cdesc()
    null = ctypes.c_void_p(0)
    assert lib.mvm_conv_silu_fwd(ctypes.byref(d), *([null] * 5)) == _lib.MVM_ERR_INVALID_ARG
    fake = ctypes.c_void_p(0x1000)
    need = lib.mvm_conv_workspace_bytes(ctypes.byref(d))
    rc = lib.mvm_conv_silu_bwd(ctypes.byref(d), *([fake] * 8), need - 1, null)
    assert rc == _lib.MVM_ERR_WORKSPACE


def _fdesc(B=2, L=40, D=24, N=16, K=3):
    fd = _lib.FusedDesc()
    fd.scan = _desc(B, L, D, N, K)
    # delta_raw (K, B, L, D); y (B, L, K, D); z a strided half of (B, L, K, 2D)
    fd.dt_stride_k, fd.dt_stride_b, fd.dt_stride_t = B * L * D, L * D, D
    fd.y_stride_b, fd.y_stride_t, fd.y_stride_k = L * K * D, K * D, D
    fd.z_stride_b, fd.z_stride_t, fd.z_stride_k = L * K * 2 * D, K * 2 * D, 2 * D
    return fd


@pytest.mark.parametrize("field,value,code", [
    ("dt_stride_t", 3, _lib.MVM_ERR_INVALID_ARG), ("y_stride_b", -1, _lib.MVM_ERR_INVALID_ARG),
    ("y_stride_b", 0, _lib.MVM_ERR_INVALID_ARG), ("dt_stride_k", 0, _lib.MVM_ERR_INVALID_ARG),
])
def test_fused_bad_descriptors_rejected(field, value, code):
    lib = _lib.lib()
    fd = _fdesc()
    assert lib.mvm_scan_fused_validate(ctypes.byref(fd)) == 0
    for which, gate in ((0, 0), (1, 0), (1, 1)):
        assert lib.mvm_scan_fused_workspace_bytes(ctypes.byref(fd), which, gate) >= 0
    setattr(fd, field, value)
    assert lib.mvm_scan_fused_validate(ctypes.byref(fd)) == code


def test_fused_a_log_flag_and_reserved_field():
    """a_is_log selects the A_log parametrisation (any value accepted, same
    workspace); the reserved field must stay 0."""
    lib = _lib.lib()
    fd = _fdesc()
    base = lib.mvm_scan_fused_workspace_bytes(ctypes.byref(fd), 1, 1)
    fd.a_is_log = 1
    assert lib.mvm_scan_fused_validate(ctypes.byref(fd)) == 0
    assert lib.mvm_scan_fused_workspace_bytes(ctypes.byref(fd), 1, 1) == base
    fd.reserved = 7
    assert lib.mvm_scan_fused_validate(ctypes.byref(fd)) == _lib.MVM_ERR_INVALID_ARG
    assert "reserved" in _lib.last_error()


def test_fused_is_float32_only():
    lib = _lib.lib()
    fd = _fdesc()
    fd.scan.in_dtype = _lib.MVM_BF16
    assert lib.mvm_scan_fused_validate(ctypes.byref(fd)) == _lib.MVM_ERR_UNSUPPORTED
    assert "float32" in _lib.last_error()


def test_fused_gate_needs_no_extra_workspace():
    """The gate's backward runs inside the scan's staging: no dense buffer."""
    lib = _lib.lib()
    fd = _fdesc()
    plain = lib.mvm_scan_fused_workspace_bytes(ctypes.byref(fd), 1, 0)
    gated = lib.mvm_scan_fused_workspace_bytes(ctypes.byref(fd), 1, 1)
    assert gated == plain > 0


def test_fused_null_pointers_rejected_before_launch():
    lib = _lib.lib()
    fd = _fdesc()
    null = ctypes.c_void_p(0)
    fake = ctypes.c_void_p(0x1000)
    # forward without y
    args = [fake] * 12
    args[8] = null
    assert lib.mvm_scan_fused_fwd(ctypes.byref(fd), *args, 0, null) == _lib.MVM_ERR_INVALID_ARG
    # backward: a gate (z) without y_raw
    bargs = [fake] * 20
    bargs[8] = fake   # z
    bargs[9] = null   # y_raw
    need = lib.mvm_scan_fused_workspace_bytes(ctypes.byref(fd), 1, 1)
    rc = lib.mvm_scan_fused_bwd(ctypes.byref(fd), *bargs, need, null)
    assert rc == _lib.MVM_ERR_INVALID_ARG
    # backward: delta_bias without ddelta_bias
    bargs = [fake] * 20
    bargs[12] = null  # ddelta_bias
    assert lib.mvm_scan_fused_bwd(ctypes.byref(fd), *bargs, need, null) == _lib.MVM_ERR_INVALID_ARG
    # backward without checkpoints
    bargs = [fake] * 20
    bargs[9 + 1] = null  # ckpt
    assert lib.mvm_scan_fused_bwd(ctypes.byref(fd), *bargs, need, null) == _lib.MVM_ERR_INVALID_ARG


def _norm_desc(rows=100, cols=384, xs=None, ys=None, eps=1e-5):
    d = _lib.NormDesc()
    d.rows, d.cols = rows, cols
    d.x_stride = cols if xs is None else xs
    d.y_stride = cols if ys is None else ys
    d.eps = eps
    d.reserved = 0
    return d


def test_norm_desc_layout_matches_header():
    # int64 x4, float, int32: 40 bytes, no padding
    assert ctypes.sizeof(_lib.NormDesc) == 40
    assert _lib.NormDesc.eps.offset == 32 and _lib.NormDesc.reserved.offset == 36


@pytest.mark.parametrize("field,value,code", [
    ("rows", -1, _lib.MVM_ERR_INVALID_ARG),
    ("rows", (1 << 25) + 1, _lib.MVM_ERR_UNSUPPORTED),
    ("cols", 0, _lib.MVM_ERR_UNSUPPORTED),
    ("cols", _lib.MVM_NORM_MAX_COLS + 1, _lib.MVM_ERR_UNSUPPORTED),
    ("x_stride", 383, _lib.MVM_ERR_INVALID_ARG),
    ("y_stride", 100, _lib.MVM_ERR_INVALID_ARG),
    ("eps", -1e-5, _lib.MVM_ERR_INVALID_ARG),
    ("eps", float("nan"), _lib.MVM_ERR_INVALID_ARG),
    ("eps", float("inf"), _lib.MVM_ERR_INVALID_ARG),
    ("reserved", 1, _lib.MVM_ERR_INVALID_ARG),
])
def test_norm_bad_descriptors_rejected(field, value, code):
    lib = _lib.lib()
    d = _norm_desc()
    assert lib.mvm_norm_validate(ctypes.byref(d)) == _lib.MVM_OK
    setattr(d, field, value)
    assert lib.mvm_norm_validate(ctypes.byref(d)) == code
    assert _lib.last_error() != ""
    assert lib.mvm_norm_workspace_bytes(ctypes.byref(d)) == code


def test_norm_workspace_and_host_checks():
    lib = _lib.lib()
    null = ctypes.c_void_p(0)
    # one partial row (2 * cols floats) per backward workgroup (8 rows per
    # workgroup pass), <= 256 of them
    for rows, blocks in ((1, 1), (16, 2), (6272, 256), (0, 1)):
        d = _norm_desc(rows=rows)
        need = lib.mvm_norm_workspace_bytes(ctypes.byref(d))
        assert need >= blocks * 2 * 384 * 4 and need % 256 == 0 and need - blocks * 2 * 384 * 4 < 256
    d = _norm_desc(rows=0)
    # an empty forward needs no buffers and launches nothing
    assert lib.mvm_layernorm_fwd(ctypes.byref(d), *([null] * 6), null) == _lib.MVM_OK
    d = _norm_desc(rows=10)
    assert lib.mvm_layernorm_fwd(ctypes.byref(d), *([null] * 6), null) == _lib.MVM_ERR_INVALID_ARG
    assert "NULL" in _lib.last_error()
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: validation fails first
    need = lib.mvm_norm_workspace_bytes(ctypes.byref(d))
    assert lib.mvm_layernorm_bwd(ctypes.byref(d), *([fake] * 10), need - 1, null) == _lib.MVM_ERR_WORKSPACE
    assert lib.mvm_layernorm_bwd(ctypes.byref(d), fake, fake, fake, fake, fake, null, fake, null, fake,
                                 fake, need, null) == _lib.MVM_ERR_INVALID_ARG


def test_fused_overlapping_gate_rejected_before_launch():
    """z strides are checked when a gate is given (without one they are 0);
    an overlapping z / dz layout fails before anything is launched."""
    lib = _lib.lib()
    fd = _fdesc()
    fd.z_stride_t = 5
    assert lib.mvm_scan_fused_validate(ctypes.byref(fd)) == 0
    fake, null = ctypes.c_void_p(0x1000), ctypes.c_void_p(0)
    need = lib.mvm_scan_fused_workspace_bytes(ctypes.byref(fd), 0, 1)
    ws = ctypes.c_void_p(0x100000)
    rc = lib.mvm_scan_fused_fwd(ctypes.byref(fd), *([fake] * 10), null, ws, need, null)
    assert rc == _lib.MVM_ERR_INVALID_ARG and "z strides" in _lib.last_error()
    need = lib.mvm_scan_fused_workspace_bytes(ctypes.byref(fd), 1, 1)
    rc = lib.mvm_scan_fused_bwd(ctypes.byref(fd), *([fake] * 19), ws, need, null)
    assert rc == _lib.MVM_ERR_INVALID_ARG and "z strides" in _lib.last_error()


def test_noalloc_backward_rejects_before_touching_the_gpu():
    """mvm_scan_bwd_noalloc: a missing checkpoint and a shape whose scratch
    need exceeds the static array fail on the host, before any device call."""
    lib = _lib.lib()
    cap = lib.mvm_scan_noalloc_scratch_bytes()
    assert cap == 64 * 1024 * 1024
    fake, null = ctypes.c_void_p(0x1000), ctypes.c_void_p(0)
    d = _desc(B=2, L=196, D=1536, N=16)
    args = [fake] * 6 + [null] + [fake] * 8
    assert lib.mvm_scan_bwd_noalloc(ctypes.byref(d), *args, null) == _lib.MVM_ERR_INVALID_ARG
    assert "ckpt" in _lib.last_error()
    big = _desc(B=8, L=16384, D=1536, N=16)
    assert lib.mvm_scan_workspace_bytes(ctypes.byref(big), 1) > cap
    rc = lib.mvm_scan_bwd_noalloc(ctypes.byref(big), *([fake] * 15), null)
    assert rc == _lib.MVM_ERR_WORKSPACE and "static array" in _lib.last_error()
    # the shapes it is sized for fit
    step = _desc(B=32, L=196, D=768, N=16, K=4)
    assert 0 < lib.mvm_scan_workspace_bytes(ctypes.byref(step), 1) <= cap
    assert lib.mvm_scan_workspace_bytes(ctypes.byref(d), 1) <= cap


def test_adamw_rejects_bad_arguments_on_the_host():
    """mvm_adamw_step validates its hyperparameters and tensor table before
    any launch (no GPU needed); an empty table is a no-op."""
    lib = _lib.lib()
    fake, null = ctypes.c_void_p(0x1000), ctypes.c_void_p(0)

    def hp(**kw):
        h = _lib.AdamwHparams()
        h.lr, h.beta1, h.beta2, h.eps, h.weight_decay, h.reserved = 1e-3, 0.9, 0.999, 1e-8, 0.01, 0
        for k, v in kw.items():
            setattr(h, k, v)
        return h

    tab = (_lib.AdamwTensor * 2)()
    for t in tab:
        t.param, t.grad, t.numel, t.state_offset = 0x1000, 0x2000, 10, 0
    good = hp()
    assert lib.mvm_adamw_step(tab, 0, ctypes.byref(good), fake, fake, fake, null) == _lib.MVM_OK
    for bad in (hp(beta1=1.0), hp(beta2=-0.1), hp(eps=0.0), hp(lr=-1.0), hp(weight_decay=-1.0),
                hp(reserved=1), hp(lr=float("nan"))):
        assert lib.mvm_adamw_step(tab, 2, ctypes.byref(bad), fake, fake, fake, null) == \
            _lib.MVM_ERR_INVALID_ARG
    assert lib.mvm_adamw_step(tab, 2, None, fake, fake, fake, null) == _lib.MVM_ERR_INVALID_ARG
    assert lib.mvm_adamw_step(tab, -1, ctypes.byref(good), fake, fake, fake, null) == \
        _lib.MVM_ERR_INVALID_ARG
    assert lib.mvm_adamw_step(None, 2, ctypes.byref(good), fake, fake, fake, null) == \
        _lib.MVM_ERR_INVALID_ARG
    assert lib.mvm_adamw_step(tab, 2, ctypes.byref(good), null, fake, fake, null) == \
        _lib.MVM_ERR_INVALID_ARG
    tab[1].numel = -5
    assert lib.mvm_adamw_step(tab, 2, ctypes.byref(good), fake, fake, fake, null) == \
        _lib.MVM_ERR_INVALID_ARG
    tab[1].numel, tab[1].grad = 10, 0
    assert lib.mvm_adamw_step(tab, 2, ctypes.byref(good), fake, fake, fake, null) == \
        _lib.MVM_ERR_INVALID_ARG
    assert "NULL param or grad" in _lib.last_error()


def test_adamw_cpu_parameters_raise_no_fallback():
    from mlx_vision_mamba_amd.optim import AdamW
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        AdamW([torch.nn.Parameter(torch.zeros(3))])
