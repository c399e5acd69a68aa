"""AdamW over all of a model's float32 parameters in one HIP kernel launch
(``mvm_adamw_step``, include/mvm_optim.h).

The update is torch.optim.AdamW's (decoupled weight decay, bias-corrected
moments), so a train step can swap ``torch.optim.AdamW(params, ...)`` for
``AdamW(params, ...)``.  The step count lives on the device and is
incremented by a device op before the kernel, so the whole step can be
captured in a HIP graph and replayed.  The first and second moments of all
tensors are two flat float32 buffers.

One difference from torch.optim.AdamW: there is a single step count for all
tensors, advanced by every ``step()``, where torch keeps one per parameter
and advances it only when that parameter has a gradient.  The two agree
when every parameter has a gradient on every step (the VisionMamba train
step); a parameter whose gradient is missing on some steps gets torch's
moments but a bias correction computed from the global count.  The count
is float32, exact up to 2^24 steps.

The tensor table (parameter and gradient pointers) is rebuilt on the host
only when a pointer changes: gradients set to None and re-created by the
next backward change it every eager step; a captured step sees the graph's
own, fixed gradient buffers.  There is no CPU path.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .scan import _stream_ptr


class AdamW:
    """One-launch AdamW for float32 CUDA parameters (same defaults as
    torch.optim.AdamW).  ``step()`` updates every parameter that has a
    gradient; ``zero_grad(set_to_none=True)`` drops the gradients."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2):
        self.params = [p for p in params if p.requires_grad]
        if not self.params:
            raise ValueError("AdamW got no parameters that require a gradient")
        dev = self.params[0].device
        if dev.type != "cuda":
            raise RuntimeError("AdamW runs only on the GPU (HIP); there is no CPU fallback")
        for p in self.params:
            if p.device != dev or p.dtype != torch.float32 or not p.is_contiguous():
                raise ValueError("AdamW takes contiguous float32 parameters on one device; got "
                                 f"{p.dtype} {tuple(p.shape)} on {p.device}")
        if not (lr >= 0 and 0 <= betas[0] < 1 and 0 <= betas[1] < 1 and eps > 0
                and weight_decay >= 0):
            raise ValueError(f"bad AdamW hyperparameters lr={lr} betas={betas} eps={eps} "
                             f"weight_decay={weight_decay}")
        self.lr, self.betas, self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self.device = dev
        self.offsets = []
        total = 0
        for p in self.params:
            self.offsets.append(total)
            total += p.numel()
        self.exp_avg = torch.zeros(total, dtype=torch.float32, device=dev)
        self.exp_avg_sq = torch.zeros(total, dtype=torch.float32, device=dev)
        self.step_count = torch.zeros(1, dtype=torch.float32, device=dev)
        self._key = None
        self._table = None
        self._n = 0

    def zero_grad(self, set_to_none: bool = True):
        for p in self.params:
            if p.grad is None:
                continue
            if set_to_none:
                p.grad = None
            else:
                p.grad.zero_()

    def _tensor_table(self):
        live = [(p, off) for p, off in zip(self.params, self.offsets) if p.grad is not None]
        key = tuple((p.data_ptr(), p.grad.data_ptr()) for p, _ in live)
        if key != self._key:
            arr = (_lib.AdamwTensor * max(1, len(live)))()
            for i, (p, off) in enumerate(live):
                g = p.grad
                if g.dtype != torch.float32 or g.shape != p.shape or not g.is_contiguous():
                    raise ValueError(f"AdamW needs contiguous float32 gradients shaped like their "
                                     f"parameters; got {g.dtype} {tuple(g.shape)}")
                arr[i].param = p.data_ptr()
                arr[i].grad = g.data_ptr()
                arr[i].numel = p.numel()
                arr[i].state_offset = off
            self._key, self._table, self._n = key, arr, len(live)
        return self._table, self._n

    @torch.no_grad()
    def step(self):
        table, n = self._tensor_table()
        if n == 0:
            return
        hp = _lib.AdamwHparams()
        hp.lr, hp.beta1, hp.beta2 = self.lr, self.betas[0], self.betas[1]
        hp.eps, hp.weight_decay, hp.reserved = self.eps, self.weight_decay, 0
        self.step_count += 1
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().mvm_adamw_step(
                table, n, ctypes.byref(hp), ctypes.c_void_p(self.step_count.data_ptr()),
                ctypes.c_void_p(self.exp_avg.data_ptr()),
                ctypes.c_void_p(self.exp_avg_sq.data_ptr()),
                ctypes.c_void_p(_stream_ptr(self.device))))
