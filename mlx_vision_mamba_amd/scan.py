"""Selective scan on MI355X: autograd Functions over the HIP C ABI.

Drop-in for the reference's scan entry points (paths relative to the
reference repository root):

* ``selective_scan(x, delta, A, B, C, D) -> y``   mamba_block.py:20-74
* ``selective_scan_chunked`` / ``selective_scan_parallel``   mamba_fast.py:17, :165
* ``selective_scan_metal`` (forward only, no autograd)       mamba_metal.py:230
* ``selective_scan_metal_trainable``                         mamba_metal.py:275
* ``selective_scan_metal_fused``                             mamba_metal_fused.py:253

All of them compute the same function with the same six gradients; they run
the HIP kernels of libmvm_scan.so and differ only in how the sequence is cut
into time chunks.  CPU tensors raise: there is no CPU fallback.

``selective_scan_directions`` is the index-remapped multi-direction form
used by the direction blocks: K scans over (B, L, K, D) token-order tensors,
where scan position s of direction k reads and writes token row
``seq_to_tok[k, s]`` (replacing the permuted copies of
mamba_block.py:254-338, :443-533).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_DT_CODE = {torch.float32: _lib.MVM_F32, torch.bfloat16: _lib.MVM_BF16}

#: scan_mode names accepted by MambaBlock (mamba_block.py:104-122) plus "hip".
SCAN_MODES = ("sequential", "chunked", "parallel", "metal", "metal_train", "metal_fused", "hip")


# Optional per-call timing: when a list, every forward / backward launch
# appends (kind, start_event, end_event, algorithmic_bytes), the events being
# recorded on the stream the kernels run on.
_timing = None


def set_scan_timing(records):
    """Start (pass a list) or stop (pass None) recording scan launches."""
    global _timing
    _timing = records


def _timer_start():
    """(records, start event) when launch timing is on, else (None, None).
    The records list is read once per call, so a call that starts recording
    also finishes it."""
    rec = _timing
    if rec is None:
        return None, None
    ev = torch.cuda.Event(enable_timing=True)
    ev.record()
    return rec, ev


def _timer_stop(rec, ev0, kind, nbytes_fn):
    if rec is not None:
        ev1 = torch.cuda.Event(enable_timing=True)
        ev1.record()
        rec.append((kind, ev0, ev1, nbytes_fn()))


def algorithmic_bytes(bsz, L, D, N, in_size, out_size, ndir=1):
    """Bytes a scan forward / VJP must move if every tensor is read or
    written exactly once: (forward, vjp).  delta, ddelta, A, dA, D, dD are
    float32; u, B, C, dy use in_size and y, du, dB, dC use out_size bytes.
    ``bsz`` counts (batch, direction) rows; A and D exist once per direction."""
    fwd = (bsz * L * D * (in_size + 4 + out_size) + bsz * L * N * 2 * in_size
           + ndir * (D * N * 4 + D * 4))
    vjp = (bsz * L * D * (in_size + 4 + in_size + out_size + 4)
           + bsz * L * N * (2 * in_size + 2 * out_size) + ndir * (D * N * 8 + D * 8))
    return fwd, vjp


def algorithmic_bytes_fused(bsz, L, D, N, ndir=1, gate=True, bias=True):
    """(forward, vjp) bytes of the fused form (float32): the plain scan's
    tensors (delta_raw / ddelta_raw in place of delta / ddelta) plus, with a
    gate, z and y_raw (written by the forward; read by the VJP, which also
    writes dz), plus the dt bias and its gradient."""
    fwd, vjp = algorithmic_bytes(bsz, L, D, N, 4, 4, ndir)
    if gate:
        fwd += bsz * L * D * (4 + 4)
        vjp += bsz * L * D * (4 + 4 + 4)
    if bias:
        fwd += ndir * D * 4
        vjp += ndir * D * 8
    return fwd, vjp


def _record(kind, u, Bm, in_dt, out_dt):
    bsz, L, K, D = u.shape
    fwd, vjp = algorithmic_bytes(bsz * K, L, D, Bm.shape[-1], _SIZE[in_dt], _SIZE[out_dt], K)
    return fwd if kind == "fwd" else vjp


_SIZE = {torch.float32: 4, torch.bfloat16: 2}


def _stream_ptr(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _check_device(*ts):
    dev = ts[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            "mlx_vision_mamba_amd scans run only on the GPU (HIP); got tensors on "
            f"{dev}. There is no CPU fallback.")
    for t in ts:
        if t is not None and t.device != dev:
            raise RuntimeError(f"all scan tensors must be on {dev}; got one on {t.device}")


def _make_desc(u, Bm, in_dt, out_dt, tok, chunk_len):
    bsz, L, K, D = u.shape
    N = Bm.shape[-1]
    d = _lib.ScanDesc()
    d.batch, d.seqlen, d.dim, d.dstate, d.ndir = bsz, L, D, N, K
    d.x_stride_b, d.x_stride_t, d.x_stride_k = u.stride(0), u.stride(1), u.stride(2)
    d.bc_stride_b, d.bc_stride_t, d.bc_stride_k = Bm.stride(0), Bm.stride(1), Bm.stride(2)
    d.seq_to_tok = tok.data_ptr() if tok is not None else None
    d.in_dtype = _DT_CODE[in_dt]
    d.out_dtype = _DT_CODE[out_dt]
    d.chunk_len = int(chunk_len)
    return d


def _resolve_chunk(L, chunk_len):
    """chunk_len: int >= 0 (0 = library heuristic) or 'whole' (one chunk)."""
    if chunk_len == "whole":
        return max(16, (L + 15) // 16 * 16)
    return int(chunk_len)


def _prepare(u, delta, A, Bm, Cm, Dv):
    """Canonicalise dtypes / layouts; shapes are (B,L,K,D), (K,D,N), (B,L,K,N), (K,D)."""
    if u.dim() != 4 or delta.shape != u.shape:
        raise ValueError(f"u and delta must be (B, L, K, D) of equal shape; got {tuple(u.shape)}, "
                         f"{tuple(delta.shape)}")
    bsz, L, K, D = u.shape
    if A.dim() != 3 or A.shape[0] != K or A.shape[1] != D:
        raise ValueError(f"A must be (K={K}, D={D}, N); got {tuple(A.shape)}")
    N = A.shape[2]
    if N < 1 or N > _lib.MVM_MAX_DSTATE:
        raise ValueError(f"d_state={N} unsupported (1..{_lib.MVM_MAX_DSTATE})")
    if Bm.shape != (bsz, L, K, N) or Cm.shape != (bsz, L, K, N):
        raise ValueError(f"B and C must be {(bsz, L, K, N)}; got {tuple(Bm.shape)}, {tuple(Cm.shape)}")
    if Dv.shape != (K, D):
        raise ValueError(f"D must be {(K, D)}; got {tuple(Dv.shape)}")
    _check_device(u, delta, A, Bm, Cm, Dv)
    in_dt = torch.bfloat16 if all(t.dtype == torch.bfloat16 for t in (u, Bm, Cm)) else torch.float32
    u = u.to(in_dt).contiguous()
    Bm = Bm.to(in_dt)
    Cm = Cm.to(in_dt)
    # B / C views (e.g. column slices of a projection output) are kept when
    # they share strides and no two elements overlap; a broadcast (stride 0)
    # layout is copied, so that dB / dC get one element per (b, t, k, n)
    if not (Bm.stride() == Cm.stride() and Bm.stride(-1) == 1 and min(Bm.stride()) >= 0
            and _no_overlap(Bm)):
        Bm, Cm = Bm.contiguous(), Cm.contiguous()
    delta = delta.to(torch.float32).contiguous()
    A = A.to(torch.float32).contiguous()
    Dv = Dv.to(torch.float32).contiguous()
    return u, delta, A, Bm, Cm, Dv, in_dt


def scan_forward(u, delta, A, Bm, Cm, Dv, tok=None, chunk_len=0, out_dtype=None, save_ckpt=False):
    """Raw forward launch (no autograd).  Returns (y, ckpt or None).

    Shapes: u, delta (B,L,K,D); A (K,D,N); Bm, Cm (B,L,K,N); Dv (K,D);
    tok (K,L) int32 on the same device or None.
    """
    u, delta, A, Bm, Cm, Dv, in_dt = _prepare(u, delta, A, Bm, Cm, Dv)
    out_dt = out_dtype or in_dt
    L = u.shape[1]
    desc = _make_desc(u, Bm, in_dt, out_dt, tok, _resolve_chunk(L, chunk_len))
    lib = _lib.lib()
    dev = u.device
    with torch.cuda.device(dev):
        y = torch.empty(u.shape, dtype=out_dt, device=dev)
        ckpt = None
        if save_ckpt:
            ckpt = torch.empty(_lib.check(lib.mvm_scan_ckpt_elems(ctypes.byref(desc))),
                               dtype=torch.float32, device=dev)
        nbytes = _lib.check(lib.mvm_scan_workspace_bytes(ctypes.byref(desc), 0))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        rec, ev0 = _timer_start()
        _lib.check(lib.mvm_scan_fwd(ctypes.byref(desc), _ptr(u), _ptr(delta), _ptr(A), _ptr(Bm),
                                    _ptr(Cm), _ptr(Dv), _ptr(y), _ptr(ckpt), _ptr(ws), nbytes,
                                    ctypes.c_void_p(_stream_ptr(dev))))
        _timer_stop(rec, ev0, "fwd", lambda: _record("fwd", u, Bm, in_dt, out_dt))
    return y, ckpt


def scan_backward(u, delta, A, Bm, Cm, Dv, dy, ckpt=None, tok=None, chunk_len=0, out_dtype=None):
    """Raw VJP launch.  Returns float32/out-dtype (du, ddelta, dA, dB, dC, dD)."""
    u, delta, A, Bm, Cm, Dv, in_dt = _prepare(u, delta, A, Bm, Cm, Dv)
    out_dt = out_dtype or in_dt
    L = u.shape[1]
    desc = _make_desc(u, Bm, in_dt, out_dt, tok, _resolve_chunk(L, chunk_len))
    lib = _lib.lib()
    dev = u.device
    dy = dy.to(in_dt).contiguous()
    if dy.shape != u.shape:
        raise ValueError(f"dy shape {tuple(dy.shape)} != {tuple(u.shape)}")
    with torch.cuda.device(dev):
        du = torch.empty(u.shape, dtype=out_dt, device=dev)
        ddelta = torch.empty(u.shape, dtype=torch.float32, device=dev)
        dA = torch.empty(A.shape, dtype=torch.float32, device=dev)
        dB = torch.empty_strided(Bm.shape, Bm.stride(), dtype=out_dt, device=dev)
        dC = torch.empty_strided(Bm.shape, Bm.stride(), dtype=out_dt, device=dev)
        dD = torch.empty(Dv.shape, dtype=torch.float32, device=dev)
        which = 1 if ckpt is not None else 2
        nbytes = _lib.check(lib.mvm_scan_workspace_bytes(ctypes.byref(desc), which))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        rec, ev0 = _timer_start()
        _lib.check(lib.mvm_scan_bwd(ctypes.byref(desc), _ptr(u), _ptr(delta), _ptr(A), _ptr(Bm),
                                    _ptr(Cm), _ptr(Dv), _ptr(ckpt), _ptr(dy), _ptr(du),
                                    _ptr(ddelta), _ptr(dA), _ptr(dB), _ptr(dC), _ptr(dD),
                                    _ptr(ws), nbytes, ctypes.c_void_p(_stream_ptr(dev))))
        _timer_stop(rec, ev0, "bwd", lambda: _record("bwd", u, Bm, in_dt, out_dt))
    return du, ddelta, dA, dB, dC, dD


# ------------------------------------------------------------- fused form

def _bkd(t):
    """(b, t, k) strides of a (B, L, K, X) view."""
    return t.stride(0), t.stride(1), t.stride(2)


def _no_overlap(t):
    """True when no two elements of t share memory: ordered by stride, each
    dimension's stride clears the span of the smaller ones."""
    span = 1
    for st, sz in sorted((st, sz) for st, sz in zip(t.stride(), t.shape) if sz != 1):
        if st < span:
            return False
        span = st * sz
    return True


def _fused_desc(u, delta_raw, Bm, y, z, tok, chunk_len, a_is_log=False):
    fd = _lib.FusedDesc()
    fd.a_is_log = int(bool(a_is_log))
    fd.scan = _make_desc(u, Bm, torch.float32, torch.float32, tok, chunk_len)
    fd.dt_stride_b, fd.dt_stride_t, fd.dt_stride_k = _bkd(delta_raw)
    fd.y_stride_b, fd.y_stride_t, fd.y_stride_k = _bkd(y)
    if z is not None:
        fd.z_stride_b, fd.z_stride_t, fd.z_stride_k = _bkd(z)
    return fd


def _check_fused(u, delta_raw, delta_bias, A, Bm, Cm, Dv, z):
    bsz, L, K, D = u.shape
    N = A.shape[-1]
    if delta_raw.shape != u.shape or (z is not None and z.shape != u.shape):
        raise ValueError("u, delta_raw and z must share the (B, L, K, D) shape")
    if A.shape != (K, D, N) or Bm.shape != (bsz, L, K, N) or Cm.shape != Bm.shape:
        raise ValueError("A must be (K, D, N) and B, C (B, L, K, N)")
    if Dv.shape != (K, D) or (delta_bias is not None and delta_bias.shape != (K, D)):
        raise ValueError("D and the dt bias must be (K, D)")
    if Bm.stride() != Cm.stride():
        raise ValueError("B and C must share strides")
    ts = [u, delta_raw, A, Bm, Cm, Dv] + [t for t in (delta_bias, z) if t is not None]
    _check_device(*ts)
    for t in ts:
        if t.dtype != torch.float32 or t.stride(-1) != 1:
            raise ValueError("the fused scan takes float32 views with channel stride 1")
    if not (A.is_contiguous() and Dv.is_contiguous()
            and (delta_bias is None or delta_bias.is_contiguous())):
        raise ValueError("A, D and the dt bias must be contiguous")


def scan_fused_forward(u, delta_raw, delta_bias, A, Bm, Cm, Dv, z, tok=None, chunk_len=0,
                       save=False, a_is_log=False):
    """y = scan(u, softplus(delta_raw + delta_bias), A, B, C, D) * silu(z)
    (mamba_block.py:180-190) in one launch sequence.  With ``a_is_log`` the
    A argument holds A_log and the kernels use A = -exp(A_log) (:184).

    u, delta_raw, z: (B, L, K, D) float32 views with channel stride 1 and any
    other strides (z may be None: no gate); delta_bias (K, D) or None;
    A (K, D, N); Bm, Cm (B, L, K, N) views; Dv (K, D).  Returns
    (y, y_raw, ckpt): y (B, L, K, D) contiguous; y_raw and ckpt are saved for
    the backward when ``save`` (else None).
    """
    _check_fused(u, delta_raw, delta_bias, A, Bm, Cm, Dv, z)
    dev = u.device
    L = u.shape[1]
    y = torch.empty(u.shape, dtype=torch.float32, device=dev)
    fd = _fused_desc(u, delta_raw, Bm, y, z, tok, _resolve_chunk(L, chunk_len), a_is_log)
    lib = _lib.lib()
    with torch.cuda.device(dev):
        y_raw = torch.empty_like(y) if (save and z is not None) else None
        ckpt = None
        if save:
            ckpt = torch.empty(_lib.check(lib.mvm_scan_ckpt_elems(ctypes.byref(fd.scan))),
                               dtype=torch.float32, device=dev)
        nbytes = _lib.check(lib.mvm_scan_fused_workspace_bytes(ctypes.byref(fd), 0, int(z is not None)))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        rec, ev0 = _timer_start()
        _lib.check(lib.mvm_scan_fused_fwd(
            ctypes.byref(fd), _ptr(u), _ptr(delta_raw), _ptr(delta_bias), _ptr(A), _ptr(Bm),
            _ptr(Cm), _ptr(Dv), _ptr(z), _ptr(y), _ptr(y_raw), _ptr(ckpt), _ptr(ws), nbytes,
            ctypes.c_void_p(_stream_ptr(dev))))
        _timer_stop(rec, ev0, "fwd", lambda: algorithmic_bytes_fused(
            u.shape[0] * u.shape[2], L, u.shape[3], A.shape[-1], u.shape[2], z is not None,
            delta_bias is not None)[0])
    return y, y_raw, ckpt


def scan_fused_backward(u, delta_raw, delta_bias, A, Bm, Cm, Dv, z, y_raw, ckpt, dy, tok=None,
                        chunk_len=0, du=None, ddelta_raw=None, dB=None, dC=None, dz=None,
                        a_is_log=False):
    """VJP of scan_fused_forward for dy (gradient of the gated y).  With
    ``a_is_log`` (A holds A_log) the returned dA is the gradient with
    respect to A_log.

    Output views may be passed in (any strides with channel stride 1, e.g.
    slices of a larger gradient buffer); missing ones are allocated with
    the layout of their primal.  Returns (du, ddelta_raw, ddelta_bias, dA,
    dB, dC, dD, dz); ddelta_bias is None without a bias, dz None without a
    gate.
    """
    _check_fused(u, delta_raw, delta_bias, A, Bm, Cm, Dv, z)
    dev = u.device
    L = u.shape[1]
    if dy.shape != u.shape:
        raise ValueError(f"dy shape {tuple(dy.shape)} != {tuple(u.shape)}")
    # dy and y_raw share the y strides of the descriptor
    ref = y_raw if (z is not None and y_raw is not None) else None
    if ref is not None and not ref.is_contiguous():
        raise ValueError("y_raw must be contiguous")
    if dy.dtype != torch.float32 or not dy.is_contiguous():
        dy = dy.float().contiguous()

    def like(t):
        # same strides as the primal (a layout with gaps allocates its span)
        if not _no_overlap(t):
            raise ValueError("a primal whose elements overlap (e.g. broadcast) needs an output view")
        return torch.empty_strided(t.shape, t.stride(), dtype=torch.float32, device=dev)

    du = like(u) if du is None else du
    ddelta_raw = like(delta_raw) if ddelta_raw is None else ddelta_raw
    if dB is None or dC is None:
        dB, dC = like(Bm), like(Bm)
    if dB.stride() != Bm.stride() or dC.stride() != Bm.stride():
        raise ValueError("dB and dC must have the strides of B")
    if z is not None and dz is None:
        dz = like(z)
    for t in (du, ddelta_raw, dB, dC) + ((dz,) if z is not None else ()):
        if not _no_overlap(t):
            raise ValueError("gradient views must not overlap themselves")
    if (z is not None and dz.stride() != z.stride()) or ddelta_raw.stride() != delta_raw.stride() \
            or du.stride() != u.stride():
        raise ValueError("gradient views must have the strides of their primals")
    ddelta_bias = torch.empty_like(delta_bias) if delta_bias is not None else None
    dA = torch.empty(A.shape, dtype=torch.float32, device=dev)
    dD = torch.empty(Dv.shape, dtype=torch.float32, device=dev)
    fd = _fused_desc(u, delta_raw, Bm, dy, z, tok, _resolve_chunk(L, chunk_len), a_is_log)
    lib = _lib.lib()
    with torch.cuda.device(dev):
        nbytes = _lib.check(lib.mvm_scan_fused_workspace_bytes(ctypes.byref(fd), 1, int(z is not None)))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        rec, ev0 = _timer_start()
        _lib.check(lib.mvm_scan_fused_bwd(
            ctypes.byref(fd), _ptr(u), _ptr(delta_raw), _ptr(delta_bias), _ptr(A), _ptr(Bm),
            _ptr(Cm), _ptr(Dv), _ptr(z), _ptr(y_raw), _ptr(ckpt), _ptr(dy), _ptr(du),
            _ptr(ddelta_raw), _ptr(ddelta_bias), _ptr(dA), _ptr(dB), _ptr(dC), _ptr(dD), _ptr(dz),
            _ptr(ws), nbytes, ctypes.c_void_p(_stream_ptr(dev))))
        _timer_stop(rec, ev0, "bwd", lambda: algorithmic_bytes_fused(
            u.shape[0] * u.shape[2], L, u.shape[3], A.shape[-1], u.shape[2], z is not None,
            delta_bias is not None)[1])
    return du, ddelta_raw, ddelta_bias, dA, dB, dC, dD, dz


class _SelectiveScanFn(torch.autograd.Function):
    """y = scan(u, delta, A, B, C, D) with the fused HIP VJP
    (the custom_function + vjp pair of mamba_metal_fused.py:229-250)."""

    @staticmethod
    def forward(ctx, u, delta, A, Bm, Cm, Dv, tok, chunk_len, out_dtype, grad_mode):
        # checkpoints only when a gradient can be asked for; grad mode is off
        # inside forward, so the caller passes its own (grad_mode)
        needs = grad_mode and any(ctx.needs_input_grad[:6])
        y, ckpt = scan_forward(u, delta, A, Bm, Cm, Dv, tok, chunk_len, out_dtype, save_ckpt=needs)
        ctx.chunk_len = chunk_len
        ctx.out_dtype = out_dtype
        ctx.in_dtypes = tuple(t.dtype for t in (u, delta, A, Bm, Cm, Dv))
        if needs:
            ctx.save_for_backward(u, delta, A, Bm, Cm, Dv, ckpt, tok)
        return y

    @staticmethod
    def backward(ctx, dy):
        u, delta, A, Bm, Cm, Dv, ckpt, tok = ctx.saved_tensors
        grads = scan_backward(u, delta, A, Bm, Cm, Dv, dy, ckpt, tok, ctx.chunk_len, ctx.out_dtype)
        grads = tuple(g.to(dt) for g, dt in zip(grads, ctx.in_dtypes))
        return grads + (None, None, None, None)


def check_permutation_table(table):
    """Raises ValueError unless every row of the (K, L) table is a
    permutation of 0..L-1.  The kernels only clamp table entries into
    [0, L): a row that misses a token would leave that token's outputs
    unwritten and a repeated token would be written twice.  The check runs
    once per table tensor (and again after an in-place change)."""
    stamp = (table.data_ptr(), table._version)
    if getattr(table, "_mvm_perm_checked", None) == stamp:
        return
    K, L = table.shape
    ok = True
    if L > 0:
        srt = torch.sort(table.long(), dim=1).values
        ok = bool((srt == torch.arange(L, device=table.device)).all())
    if not ok:
        raise ValueError("seq_to_tok: every row must be a permutation of 0..L-1")
    table._mvm_perm_checked = stamp


def selective_scan_directions(u, delta, A, B, C, D, seq_to_tok=None, chunk_len=0, out_dtype=None,
                              forward_only=False):
    """K index-remapped scans in one launch.

    u, delta: (B, L, K, D) in token order; A: (K, D, N); B, C: (B, L, K, N);
    D: (K, D); seq_to_tok: (K, L) int32 tensor on the GPU (or None for the
    identity order).  Returns y (B, L, K, D) in token order.
    ``forward_only`` returns a detached y without saving checkpoints (the
    reference's inference-only ``metal`` mode).
    """
    if seq_to_tok is not None:
        if seq_to_tok.dtype != torch.int32 or seq_to_tok.shape != (u.shape[2], u.shape[1]):
            raise ValueError("seq_to_tok must be int32 of shape (K, L)")
        # checked on the caller's tensor, so that a table kept on the host is
        # checked once, not again for every fresh device copy
        check_permutation_table(seq_to_tok)
        seq_to_tok = seq_to_tok.to(u.device).contiguous()
    if forward_only:
        y, _ = scan_forward(u.detach(), delta.detach(), A.detach(), B.detach(), C.detach(),
                            D.detach(), seq_to_tok, _resolve_chunk(u.shape[1], chunk_len), out_dtype)
        return y
    return _apply_scan(u, delta, A, B, C, D, seq_to_tok, chunk_len, out_dtype)


def _apply_scan(u, delta, A, B, C, D, tok, chunk_len, out_dtype):
    """_SelectiveScanFn.apply, saving checkpoints only when grad mode is on
    (not under torch.no_grad / inference_mode)."""
    return _SelectiveScanFn.apply(u, delta, A, B, C, D, tok, chunk_len, out_dtype,
                                  torch.is_grad_enabled())


def _scan3(x, delta, A, B, C, D, chunk_len, out_dtype=None):
    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, D); got {tuple(x.shape)}")
    y = _apply_scan(x.unsqueeze(2), delta.unsqueeze(2), A.unsqueeze(0), B.unsqueeze(2),
                    C.unsqueeze(2), D.unsqueeze(0), None, chunk_len, out_dtype)
    return y.squeeze(2)


def selective_scan(x, delta, A, B, C, D, chunk_len=0, out_dtype=None):
    """Selective scan (S6), forward + VJP on the GPU.  mamba_block.py:20-74.

    x, delta: (B, L, D_inner); A: (D_inner, N); B, C: (B, L, N); D: (D_inner,).
    ``chunk_len`` = 0 lets the library cut long sequences into time chunks
    (two-pass carry); ``"whole"`` keeps one chunk per channel.
    """
    return _scan3(x, delta, A, B, C, D, chunk_len, out_dtype)


def selective_scan_sequential(x, delta, A, B, C, D):
    """Sequential in time: one chunk per channel (the ``sequential`` mode)."""
    return _scan3(x, delta, A, B, C, D, "whole")


def selective_scan_chunked(x, delta, A, B, C, D, chunk_size=32):
    """mamba_fast.py:17 ``chunked`` mode: time chunks of ``chunk_size``
    (rounded up to a multiple of 16) joined by the carry pass."""
    return _scan3(x, delta, A, B, C, D, max(16, (int(chunk_size) + 15) // 16 * 16))


def selective_scan_parallel(x, delta, A, B, C, D):
    """mamba_fast.py:165 ``parallel`` mode: chunk-parallel scan, chunk
    length chosen by the library."""
    return _scan3(x, delta, A, B, C, D, 0)


def selective_scan_metal(x, delta, A, B, C, D):
    """mamba_metal.py:230 ``metal`` mode: inference only, no autograd (the
    result is detached and no checkpoints are written)."""
    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, D); got {tuple(x.shape)}")
    y, _ = scan_forward(x.detach().unsqueeze(2), delta.detach().unsqueeze(2), A.detach().unsqueeze(0),
                        B.detach().unsqueeze(2), C.detach().unsqueeze(2), D.detach().unsqueeze(0))
    return y.squeeze(2)


def selective_scan_metal_trainable(x, delta, A, B, C, D):
    """mamba_metal.py:275 ``metal_train`` mode (same function and gradients)."""
    return _scan3(x, delta, A, B, C, D, 0)


def selective_scan_metal_fused(x, delta, A, B, C, D):
    """mamba_metal_fused.py:253 ``metal_fused`` mode."""
    return _scan3(x, delta, A, B, C, D, 0)


_MODE_FNS = {
    "sequential": selective_scan_sequential,
    "chunked": selective_scan_chunked,
    "parallel": selective_scan_parallel,
    "metal": selective_scan_metal,
    "metal_train": selective_scan_metal_trainable,
    "metal_fused": selective_scan_metal_fused,
    "hip": selective_scan,
}

# chunk_len used by the direction blocks for each mode
_MODE_CHUNK = {"sequential": "whole", "chunked": 32, "parallel": 0, "metal": 0,
               "metal_train": 0, "metal_fused": 0, "hip": 0}


def get_scan_fn(scan_mode: str):
    """Scan function for a scan_mode string (mamba_block.py:104-122).

    Unknown names raise ValueError (the reference silently fell back to the
    sequential scan, mamba_block.py:121-122).
    """
    try:
        return _MODE_FNS[scan_mode]
    except KeyError:
        raise ValueError(f"unknown scan_mode {scan_mode!r}; expected one of {SCAN_MODES}") from None


def chunk_len_for(rows, L, D, N=16):
    """Time-chunk length the library picks for `rows` = batch x directions
    scans of length L over D channels (the whole sequence when it is one
    chunk)."""
    d = _lib.ScanDesc()
    d.batch, d.seqlen, d.dim, d.dstate, d.ndir = rows, L, D, N, 1
    d.x_stride_b, d.x_stride_k, d.x_stride_t = L * D, 0, D
    d.bc_stride_b, d.bc_stride_k, d.bc_stride_t = L * N, 0, N
    d.in_dtype = d.out_dtype = _lib.MVM_F32
    return _lib.check(_lib.lib().mvm_scan_chunk_len(ctypes.byref(d)))


def mode_chunk_len(scan_mode: str):
    get_scan_fn(scan_mode)
    return _MODE_CHUNK[scan_mode]


def selftest_lanes(device="cuda"):
    """Runs the cross-lane layout check kernel; returns a (128,) float tensor."""
    out = torch.empty(128, dtype=torch.float32, device=device)
    with torch.cuda.device(out.device):
        _lib.check(_lib.lib().mvm_selftest_lanes(_ptr(out), ctypes.c_void_p(_stream_ptr(out.device))))
    return out
