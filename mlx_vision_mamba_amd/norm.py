"""LayerNorm over the last axis on the GPU (HIP kernels behind include/mvm_norm.h).

Replaces the reference's ``nn.LayerNorm(d_model)`` (MLX, eps 1e-5, affine):
the pre-norm of ResidualMambaBlock / BidirectionalMambaBlock /
MultiDirectionalMambaBlock (reference mamba_block.py:201-205, :222-227,
:401, :548) and the encoder's final norm (vision_mamba.py:192, :223).  The
modules keep their ``nn.LayerNorm`` children (same parameters and state_dict
keys); only the computation runs here.

``layer_norm(x, norm, residual=True)`` also returns x itself as a second
output for the block's residual branch ``x + f(norm(x))``.  The gradient
that reaches x through that branch then arrives in this function's backward
together with the normalised branch's, and the backward kernel adds the two
in its store, so no separate accumulation pass runs.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .scan import _check_device, _ptr, _stream_ptr


def _desc(rows, cols, x_stride, y_stride, eps):
    d = _lib.NormDesc()
    d.rows, d.cols, d.x_stride, d.y_stride = rows, cols, x_stride, y_stride
    d.eps = float(eps)
    d.reserved = 0
    return d


class _LayerNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, eps, residual):
        _check_device(x, weight, bias)
        E = x.shape[-1]
        if weight.shape != (E,) or bias.shape != (E,):
            raise ValueError(f"weight and bias must be ({E},); got {tuple(weight.shape)}, "
                             f"{tuple(bias.shape)}")
        x2 = x.reshape(-1, E).float().contiguous()
        w = weight.float().contiguous()
        b = bias.float().contiguous()
        R = x2.shape[0]
        dev = x.device
        y = torch.empty((R, E), dtype=torch.float32, device=dev)
        mean = torch.empty(R, dtype=torch.float32, device=dev)
        rstd = torch.empty(R, dtype=torch.float32, device=dev)
        desc = _desc(R, E, E, E, eps)
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().mvm_layernorm_fwd(ctypes.byref(desc), _ptr(x2), _ptr(w), _ptr(b),
                                                    _ptr(y), _ptr(mean), _ptr(rstd),
                                                    ctypes.c_void_p(_stream_ptr(dev))))
        ctx.save_for_backward(x2, w, mean, rstd)
        ctx.eps = eps
        ctx.shape, ctx.dtype = x.shape, x.dtype
        ctx.pdtypes = (weight.dtype, bias.dtype)
        y = y.view(x.shape).to(x.dtype)
        if residual:
            # x itself: autograd returns an alias whose gradient comes back here
            return y, x
        return y

    @staticmethod
    def backward(ctx, dy, dres=None):
        x2, w, mean, rstd = ctx.saved_tensors
        R, E = x2.shape
        dev = x2.device
        dy2 = dy.reshape(R, E).float().contiguous()
        dres2 = dres.reshape(R, E).float().contiguous() if dres is not None else None
        dx = torch.empty((R, E), dtype=torch.float32, device=dev)
        dw = torch.empty(E, dtype=torch.float32, device=dev)
        db = torch.empty(E, dtype=torch.float32, device=dev)
        desc = _desc(R, E, E, E, ctx.eps)
        lib = _lib.lib()
        with torch.cuda.device(dev):
            nbytes = _lib.check(lib.mvm_norm_workspace_bytes(ctypes.byref(desc)))
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
            _lib.check(lib.mvm_layernorm_bwd(ctypes.byref(desc), _ptr(x2), _ptr(w), _ptr(mean),
                                             _ptr(rstd), _ptr(dy2), _ptr(dres2), _ptr(dx), _ptr(dw),
                                             _ptr(db), _ptr(ws), nbytes,
                                             ctypes.c_void_p(_stream_ptr(dev))))
        return (dx.view(ctx.shape).to(ctx.dtype), dw.to(ctx.pdtypes[0]), db.to(ctx.pdtypes[1]),
                None, None)


def layer_norm(x, norm, residual=False):
    """``norm(x)`` for an ``nn.LayerNorm`` over the last axis, computed by the
    HIP kernels.  With ``residual=True`` returns ``(norm(x), x_alias)``;
    use ``x_alias`` (it is x) for the block's residual sum so that both
    gradients of x are combined by the norm's backward kernel."""
    if not isinstance(norm, torch.nn.LayerNorm):
        raise TypeError(f"layer_norm needs an nn.LayerNorm, got {type(norm).__name__}")
    if len(norm.normalized_shape) != 1 or not norm.elementwise_affine or norm.bias is None:
        raise ValueError("layer_norm supports an affine LayerNorm over the last axis with bias")
    return _LayerNormFn.apply(x, norm.weight, norm.bias, norm.eps, residual)
