"""Causal depthwise conv1d + SiLU along scan orders, on the GPU.

Replaces MambaBlock's ``conv1d`` + ``[:, :L]`` + ``silu``
(reference mamba_block.py:129-132, :170-171) for all K directions of a
block at once: x is (B, N, K, D) in token order and position s of direction
k reads token row ``seq_to_tok[k, s]``, so no permuted copy is built.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .scan import _check_device, _ptr, _stream_ptr


def _desc(x, y_strides, kc, tok, dx_strides=None):
    """Conv descriptor; strides are given in (b, t, k) order of a (B, N, K, D)
    view.  dx uses y's strides unless given."""
    bsz, L, K, D = x.shape
    d = _lib.ConvDesc()
    d.batch, d.seqlen, d.dim, d.ndir, d.kwidth = bsz, L, D, K, kc
    d.x_stride_b, d.x_stride_t, d.x_stride_k = x.stride(0), x.stride(1), x.stride(2)
    d.y_stride_b, d.y_stride_t, d.y_stride_k = y_strides[0], y_strides[1], y_strides[2]
    dxs = dx_strides if dx_strides is not None else y_strides
    d.dx_stride_b, d.dx_stride_t, d.dx_stride_k = dxs[0], dxs[1], dxs[2]
    d.seq_to_tok = tok.data_ptr() if tok is not None else None
    return d


def conv_silu_forward_into(x, w, b, y, tok):
    """Raw forward launch: y (a (B, N, K, D) view with channel stride 1, any
    other strides) = silu(conv(x) + b) along each direction's scan order."""
    K, D, kc = w.shape
    desc = _desc(x, y.stride(), kc, tok)
    with torch.cuda.device(x.device):
        _lib.check(_lib.lib().mvm_conv_silu_fwd(ctypes.byref(desc), _ptr(x), _ptr(w), _ptr(b),
                                                _ptr(y), ctypes.c_void_p(_stream_ptr(x.device))))


def conv_silu_backward_into(x, w, b, dy, dx, tok):
    """Raw backward launch: writes dx (a view with its own strides, e.g. a
    slice of a larger gradient buffer) and returns (dw, dbias)."""
    K, D, kc = w.shape
    dw = torch.empty_like(w)
    db = torch.empty_like(b)
    desc = _desc(x, dy.stride(), kc, tok, dx.stride())
    lib = _lib.lib()
    with torch.cuda.device(x.device):
        nbytes = _lib.check(lib.mvm_conv_workspace_bytes(ctypes.byref(desc)))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
        _lib.check(lib.mvm_conv_silu_bwd(ctypes.byref(desc), _ptr(x), _ptr(w), _ptr(b), _ptr(dy),
                                         _ptr(dx), _ptr(dw), _ptr(db), _ptr(ws), nbytes,
                                         ctypes.c_void_p(_stream_ptr(x.device))))
    return dw, db


class _ConvSiluFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, b, tok):
        _check_device(x, w, b)
        if x.dim() != 4 or x.stride(-1) != 1:
            x = x.contiguous()
        x = x.float()
        K, D, kc = w.shape
        w = w.float().contiguous()
        b = b.float().contiguous()
        y = torch.empty(x.shape, dtype=torch.float32, device=x.device)
        desc = _desc(x, y.stride(), kc, tok)
        with torch.cuda.device(x.device):
            _lib.check(_lib.lib().mvm_conv_silu_fwd(ctypes.byref(desc), _ptr(x), _ptr(w), _ptr(b),
                                                    _ptr(y), ctypes.c_void_p(_stream_ptr(x.device))))
        ctx.save_for_backward(x, w, b, tok)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, b, tok = ctx.saved_tensors
        K, D, kc = w.shape
        dy = dy.float().contiguous()
        dx = torch.empty(x.shape, dtype=torch.float32, device=x.device)
        dw = torch.empty_like(w)
        db = torch.empty_like(b)
        desc = _desc(x, dx.stride(), kc, tok)
        lib = _lib.lib()
        with torch.cuda.device(x.device):
            nbytes = _lib.check(lib.mvm_conv_workspace_bytes(ctypes.byref(desc)))
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
            _lib.check(lib.mvm_conv_silu_bwd(ctypes.byref(desc), _ptr(x), _ptr(w), _ptr(b), _ptr(dy),
                                             _ptr(dx), _ptr(dw), _ptr(db), _ptr(ws), nbytes,
                                             ctypes.c_void_p(_stream_ptr(x.device))))
        return dx, dw, db, None


def causal_conv_silu(x, weight, bias, seq_to_tok=None):
    """silu(causal depthwise conv) per direction.

    x: (B, N, K, D) float32 (channel stride 1, any other strides);
    weight: (K, D, d_conv); bias: (K, D); seq_to_tok: (K, N) int32 GPU
    tensor or None (identity order).  Returns (B, N, K, D) contiguous.
    """
    if weight.dim() != 3 or weight.shape[:2] != (x.shape[2], x.shape[3]):
        raise ValueError(f"weight must be (K, D, d_conv); got {tuple(weight.shape)}")
    if bias.shape != (x.shape[2], x.shape[3]):
        raise ValueError(f"bias must be (K, D); got {tuple(bias.shape)}")
    if seq_to_tok is not None:
        if seq_to_tok.dtype != torch.int32 or seq_to_tok.shape != (x.shape[2], x.shape[1]):
            raise ValueError("seq_to_tok must be int32 of shape (K, N)")
        seq_to_tok = seq_to_tok.to(x.device).contiguous()
    return _ConvSiluFn.apply(x, weight, bias, seq_to_tok)
