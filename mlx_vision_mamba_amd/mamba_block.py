"""Mamba blocks on MI355X (PyTorch modules over the HIP selective scan).

Mirrors the reference's module API (mlx_vision_mamba/mamba_block.py):
``MambaBlock`` (:77-192), ``ResidualMambaBlock`` (:195-205),
``BidirectionalMambaBlock`` (:208-237) and ``MultiDirectionalMambaBlock``
(:341-566), with the same constructor arguments, parameter names and
forward semantics, and with ``scan_mode`` passed down to every inner block
(the reference built the inner blocks with the default mode, :202, :223-224,
:403).

Direction blocks do not build permuted copies.  All K directions run as one
batch: one in_proj GEMM (E -> K*2*D_inner), a causal depthwise conv and the
selective scan that read and write through per-direction index tables, the
per-token projections batched over K, and one out_proj GEMM over the
concatenated K*D_inner features, which is also the (atomic-free) sum over
directions (:562-566).

Between the two GEMMs the block core (conv + SiLU, x_proj, dt_proj, and the
scan with the softplus of delta and the y * silu(z) gate fused into it,
:170-190) is one autograd Function whose backward writes the gradient of
the in_proj output in place: the conv's dx and the gate's dz land in the two
halves of one buffer, so no slice / cat / elementwise pass is materialised.
Activations between the projections are kept direction-major,
(K, B*N, features), so the x_proj / dt_proj GEMMs batch over K without
copies.

The direction blocks' per-direction parameters (in_proj, conv1d, x_proj,
dt_proj, A_log, D, out_proj) are slices of one (K, ...) buffer per kind owned
by the direction module, so the batched operands are views, not per-step
concatenations (out_proj's (E, K*D_inner) operand is one reordering copy);
each buffer's gradient returns to the K parameters as its K
slices.  The buffers are (re)built at the first forward and whenever a
parameter stops being its slice (after ``.to()``, or a replaced parameter).
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import directions as _dirs
from .conv import causal_conv_silu, conv_silu_backward_into, conv_silu_forward_into
from .norm import layer_norm
from .scan import (check_permutation_table, get_scan_fn, mode_chunk_len, scan_fused_backward,
                   scan_fused_forward)


def _dt_bias_init(d_inner: int, dt_min: float = 1e-3, dt_max: float = 1e-1) -> torch.Tensor:
    """dt_proj bias with softplus(bias) log-uniform in [dt_min, dt_max]."""
    dt = torch.exp(torch.rand(d_inner) * (math.log(dt_max) - math.log(dt_min)) + math.log(dt_min))
    return dt + torch.log(-torch.expm1(-dt))


class MambaBlock(nn.Module):
    """in_proj -> causal depthwise conv1d -> SiLU -> selective scan -> gate ->
    out_proj (mamba_block.py:77-192).  Input / output (B, L, d_model).

    scan_mode: "sequential", "chunked", "parallel", "metal", "metal_train",
    "metal_fused" (the reference's names, mamba_block.py:104-120) or "hip";
    every mode runs the HIP scan.  Unknown names raise ValueError.

    ``self._scan_fn`` is the scan function the mode selects
    (mamba_block.py:104-122).  The library's modes run inside the fused
    block core; a caller that assigns another callable
    ``f(x, delta, A, B, C, D) -> y`` to ``_scan_fn`` gets the reference's op
    sequence with ``f`` called where the reference calls it (:187), in this
    block and in the direction blocks that contain it.
    """

    def __init__(self, d_model: int = 384, d_state: int = 16, d_conv: int = 4,
                 expand_factor: int = 2, scan_mode: str = "sequential"):
        super().__init__()
        self.d_model = d_model
        self.d_state = d_state
        self.d_inner = d_model * expand_factor
        self.d_conv = d_conv
        self.scan_mode = scan_mode
        self._scan_fn = get_scan_fn(scan_mode)
        self.dt_rank = math.ceil(d_model / 16)                                 # :136
        self.in_proj = nn.Linear(d_model, 2 * self.d_inner, bias=False)        # :125
        self.conv1d = nn.Conv1d(self.d_inner, self.d_inner, kernel_size=d_conv,
                                padding=d_conv - 1, groups=self.d_inner)        # :129-132
        self.x_proj = nn.Linear(self.d_inner, self.dt_rank + 2 * d_state, bias=False)  # :137
        self.dt_proj = nn.Linear(self.dt_rank, self.d_inner, bias=True)        # :140
        with torch.no_grad():
            self.dt_proj.bias.copy_(_dt_bias_init(self.d_inner))
        A = torch.arange(1, d_state + 1, dtype=torch.float32).repeat(self.d_inner, 1)
        self.A_log = nn.Parameter(torch.log(A))                                # :143-147
        self.D = nn.Parameter(torch.ones(self.d_inner))                        # :150
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=False)           # :153

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if _custom_scan(self):
            return _scan_fn_forward(self, x)
        return _directional_forward([self], x, None, self.scan_mode)


class ResidualMambaBlock(nn.Module):
    """Pre-norm MambaBlock with a residual (mamba_block.py:195-205)."""

    def __init__(self, d_model: int = 384, d_state: int = 16, d_conv: int = 4,
                 expand_factor: int = 2, scan_mode: str = "sequential"):
        super().__init__()
        self.norm = nn.LayerNorm(d_model)
        self.mamba = MambaBlock(d_model, d_state, d_conv, expand_factor, scan_mode)

    def forward(self, x):
        h, xr = layer_norm(x, self.norm, residual=True)
        return xr + self.mamba(h)


class BidirectionalMambaBlock(nn.Module):
    """Forward + reversed-sequence MambaBlocks, summed with a residual
    (mamba_block.py:208-237)."""

    def __init__(self, d_model: int = 384, d_state: int = 16, d_conv: int = 4,
                 expand_factor: int = 2, scan_mode: str = "sequential"):
        super().__init__()
        self.norm = nn.LayerNorm(d_model)
        self.forward_mamba = MambaBlock(d_model, d_state, d_conv, expand_factor, scan_mode)
        self.backward_mamba = MambaBlock(d_model, d_state, d_conv, expand_factor, scan_mode)
        self.scan_mode = scan_mode
        self._tables = {}

    def forward(self, x):
        h, xr = layer_norm(x, self.norm, residual=True)                      # :227
        tok = _cached_table(self._tables, 2, x.shape[1], None, x.device)
        blocks = [self.forward_mamba, self.backward_mamba]
        if any(_custom_scan(b) for b in blocks):
            return xr + _per_direction_forward(blocks, h, tok)
        return xr + _directional_forward(blocks, h, tok, self.scan_mode,
                                         _direction_stacks(self, blocks))


class MultiDirectionalMambaBlock(nn.Module):
    """K independent MambaBlocks, one per scan order, summed with a residual
    (mamba_block.py:341-566).  K = 2, 4 (2D grid), 6 (3D) or 8 (4D).

    When the token count differs from the grid size (a subset of patches),
    the block falls back to forward + backward scans with blocks 0 and 1
    (mamba_block.py:554-559).
    """

    def __init__(self, d_model: int = 384, d_state: int = 16, d_conv: int = 4,
                 expand_factor: int = 2, num_directions: int = 2,
                 grid_shape: Optional[Sequence[int]] = None, scan_mode: str = "sequential"):
        super().__init__()
        if num_directions not in (2, 4, 6, 8):
            raise ValueError(f"num_directions must be 2, 4, 6, or 8, got {num_directions}")
        need = {4: 2, 6: 3, 8: 4}.get(num_directions)
        if need is not None and (grid_shape is None or len(grid_shape) != need):
            raise ValueError(f"K={num_directions} requires a {need}-D grid_shape, got {grid_shape}")
        self.num_directions = num_directions
        self.grid_shape = tuple(grid_shape) if grid_shape is not None else None
        self.scan_mode = scan_mode
        self.norm = nn.LayerNorm(d_model)
        self.mamba_blocks = nn.ModuleList(
            [MambaBlock(d_model, d_state, d_conv, expand_factor, scan_mode)
             for _ in range(num_directions)])
        self._tables = {}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        bsz, n, _ = x.shape
        h, xr = layer_norm(x, self.norm, residual=True)                      # :548
        expected = math.prod(self.grid_shape) if self.grid_shape is not None else n
        if n != expected and self.num_directions > 2:                         # :554-559
            tok = _cached_table(self._tables, 2, n, None, x.device)
            blocks = [self.mamba_blocks[0], self.mamba_blocks[1]]
        else:
            grid = self.grid_shape if self.num_directions > 2 else None
            tok = _cached_table(self._tables, self.num_directions, n, grid, x.device)
            blocks = list(self.mamba_blocks)
        if any(_custom_scan(b) for b in blocks):
            return xr + _per_direction_forward(blocks, h, tok)
        stacks = _direction_stacks(self, list(self.mamba_blocks))
        return xr + _directional_forward(blocks, h, tok, self.scan_mode, stacks)  # :562-566


# per-direction parameters stored as slices of one (K, ...) buffer per kind
STACKED_PARAMS = ("in_proj.weight", "conv1d.weight", "conv1d.bias", "x_proj.weight",
                  "dt_proj.weight", "dt_proj.bias", "A_log", "D", "out_proj.weight")


_STACKED_PATHS = tuple((tuple(n.split(".")[:-1]), n.split(".")[-1]) for n in STACKED_PARAMS)


def _param(blk, path):
    """The parameter at dotted ``path`` of ``blk``, by direct registry lookups
    (the same objects attribute access returns, without Module.__getattr__)."""
    *mods, name = path.split(".")
    for m in mods:
        blk = blk._modules[m]
    return blk._parameters[name]


def _params_of(blocks):
    """STACKED_PARAMS of each block, kind-major: [[kind 0 of block 0, ...], ...]."""
    out = []
    for mods, name in _STACKED_PATHS:
        row = []
        for b in blocks:
            for m in mods:
                b = b._modules[m]
            row.append(b._parameters[name])
        out.append(row)
    return out


def _is_slice_of(p, buf, k):
    return (p.device == buf.device and p.dtype == buf.dtype and p.shape == buf.shape[1:]
            and p.is_contiguous()
            and p.data_ptr() == buf.data_ptr() + k * buf.stride(0) * buf.element_size())


def _direction_stacks(owner, blocks):
    """The (K, ...) buffers whose k-th slices are the parameters of blocks[k],
    one per name of STACKED_PARAMS, kept on ``owner``.  Rebuilt (values
    copied from the current parameters, which then become slices of the new
    buffers) when any parameter is not its slice.  The per-call check
    compares each parameter's data pointer, shape and dtype with those its
    slice was given (the buffers are held here, so their memory is never
    reused while the pointers are compared)."""
    params = _params_of(blocks)
    cache = owner.__dict__.get("_param_stacks")
    if cache is not None:
        bufs, expect = cache
        flat = [p for ps in params for p in ps]
        if len(flat) == len(expect) and all(
                p.data_ptr() == ptr and p.dtype is dt and p.shape == shp
                for p, (ptr, dt, shp) in zip(flat, expect)):
            return bufs
    with torch.no_grad():
        bufs = [torch.stack([p.detach() for p in ps], 0) for ps in params]
        for buf, ps in zip(bufs, params):
            for k, p in enumerate(ps):
                p.data = buf[k]
    expect = [(p.data_ptr(), p.dtype, p.shape) for ps in params for p in ps]
    owner.__dict__["_param_stacks"] = (bufs, expect)
    return bufs


class _DirectionParams(torch.autograd.Function):
    """(buffers..., parameters...) -> the buffers, differentiable w.r.t. the
    parameters that are their slices: the backward hands each buffer's
    gradient to its K parameters as K contiguous slices (a gradient that
    arrives strided, as out_proj's does, is made contiguous once, so the
    parameters take their slices without a copy each)."""

    @staticmethod
    def forward(ctx, nbuf, *tensors):
        ctx.nbuf = nbuf
        ctx.K = tensors[0].shape[0]
        return tuple(t.view_as(t) for t in tensors[:nbuf])

    @staticmethod
    def backward(ctx, *grads):
        out = [None] * (1 + ctx.nbuf)
        for g in grads:
            out += list(g.contiguous().unbind(0)) if g is not None else [None] * ctx.K
        return tuple(out)


def _cached_table(cache, K, n, grid, device):
    key = (K, n, grid, str(device))
    if key not in cache:
        table = _dirs.seq_to_tok_table(K, n, grid).to(device)
        check_permutation_table(table)
        cache[key] = table
    return cache[key]


def _bnkd(t_kbnd, bsz, n):
    """(B, N, K, X) view of a direction-major (K, B*N, X) tensor."""
    K, _, X = t_kbnd.shape
    return t_kbnd.view(K, bsz, n, X).permute(1, 2, 0, 3)


class _MambaCoreFn(torch.autograd.Function):
    """xz (B, N, K, 2*D_inner) from in_proj -> gated scan output (B, N, K, D_inner).

    Forward (mamba_block.py:166-190, all K directions at once):
      xc    = silu(causal depthwise conv(x) + conv_b)      along each scan order
      dbc   = x_proj(xc)                                   (K, B*N, R + 2N)
      delta = softplus(dt_proj(dbc[:R]) + dt_bias)         inside the scan
      y     = scan(xc, delta, -exp(A_log), B, C, D) * silu(z)
    The scan kernels take A_log and form A = -exp(A_log) themselves; their
    dA output is the gradient of A_log.
    """

    @staticmethod
    def forward(ctx, xz, conv_w, conv_b, W_x, W_dt, b_dt, A_log, Dv, tok, chunk_len, save):
        bsz, n, K, d2 = xz.shape
        din = d2 // 2
        R = W_dt.shape[2]
        ns = A_log.shape[2]
        dev = xz.device
        xb, z = xz[..., :din], xz[..., din:]
        xc = torch.empty(K, bsz * n, din, dtype=torch.float32, device=dev)
        conv_silu_forward_into(xb, conv_w, conv_b, _bnkd(xc, bsz, n), tok)       # :170-171
        # float32 operands: the GEMMs take the weights' transposed views as they are
        dbc = torch.bmm(xc, W_x.transpose(1, 2))                                   # :174
        dt = dbc[..., :R]
        delta_raw = torch.bmm(dt, W_dt.transpose(1, 2))                            # :180
        bc = _bnkd(dbc, bsz, n)
        # save: checkpoints and y_raw are kept for the backward (training);
        # off for the forward-only mode and under no_grad / inference_mode
        y, y_raw, ckpt = scan_fused_forward(_bnkd(xc, bsz, n), _bnkd(delta_raw, bsz, n), b_dt, A_log,
                                            bc[..., R:R + ns], bc[..., R + ns:], Dv, z, tok,
                                            chunk_len, save=save, a_is_log=True)   # :181-190
        if save:
            ctx.save_for_backward(xz, conv_w, conv_b, W_x, W_dt, b_dt, A_log, Dv, tok, xc, dbc,
                                  delta_raw, y_raw, ckpt)
            ctx.chunk_len = chunk_len
        return y

    @staticmethod
    def backward(ctx, dy):
        (xz, conv_w, conv_b, W_x, W_dt, b_dt, A_log, Dv, tok, xc, dbc, delta_raw, y_raw,
         ckpt) = ctx.saved_tensors
        bsz, n, K, d2 = xz.shape
        din = d2 // 2
        R = W_dt.shape[2]
        ns = A_log.shape[2]
        dev = xz.device
        xb, z = xz[..., :din], xz[..., din:]
        dxz = torch.empty(xz.shape, dtype=torch.float32, device=dev)
        d_dbc = torch.empty_like(dbc)
        du = torch.empty_like(xc)
        ddelta_raw = torch.empty_like(delta_raw)
        bc, dbc_v = _bnkd(dbc, bsz, n), _bnkd(d_dbc, bsz, n)
        _, _, db_dt, dA_log, _, _, dDv, _ = scan_fused_backward(
            _bnkd(xc, bsz, n), _bnkd(delta_raw, bsz, n), b_dt, A_log, bc[..., R:R + ns],
            bc[..., R + ns:], Dv, z, y_raw, ckpt, dy, tok, ctx.chunk_len,
            du=_bnkd(du, bsz, n), ddelta_raw=_bnkd(ddelta_raw, bsz, n),
            dB=dbc_v[..., R:R + ns], dC=dbc_v[..., R + ns:], dz=dxz[..., din:], a_is_log=True)
        # dt_proj: delta_raw = dt @ W_dt^T; the GEMM writes the first R columns
        # of d_dbc in place (row stride R + 2N is a valid leading dimension)
        torch.bmm(ddelta_raw, W_dt, out=d_dbc[..., :R])
        dW_dt = torch.bmm(ddelta_raw.transpose(1, 2), dbc[..., :R])
        # x_proj: dbc = xc @ W_x^T; the scan's du joins through the GEMM's beta
        # (in place: du is this backward's own buffer, so no copy of it is made)
        dxc = du.baddbmm_(d_dbc, W_x)
        dW_x = _tn_split_rows(d_dbc, xc)
        # conv + SiLU: dx lands in the first half of dxz
        dconv_w, dconv_b = conv_silu_backward_into(xb, conv_w, conv_b, _bnkd(dxc, bsz, n),
                                                   dxz[..., :din], tok)
        return dxz, dconv_w, dconv_b, dW_x, dW_dt, db_dt, dA_log, dDv, None, None, None


def _tn_split_rows(a, b, splits=8):
    """a^T @ b per direction for a (K, M, P) and b (K, M, Q) with a long row
    reduction (M = B*N) and small outputs: the rows are split into ``splits``
    chunks, one batched GEMM over K*splits computes the partial products and
    they are summed in a fixed order (deterministic).  The split keeps enough
    workgroups in flight to stream b from HBM."""
    K, M, P = a.shape
    if M % splits or M // splits < 256:
        return torch.bmm(a.transpose(1, 2), b)
    m = M // splits
    part = torch.bmm(a.reshape(K * splits, m, P).transpose(1, 2), b.reshape(K * splits, m, -1))
    return part.view(K, splits, P, -1).sum(1)


def _custom_scan(blk):
    """True when the caller replaced ``blk._scan_fn`` with a function other
    than the one its ``scan_mode`` selects (mamba_block.py:104-122).  The
    library's own modes all compute the same scan, which the fused block
    core runs; any other callable is honoured by _scan_fn_forward."""
    return blk._scan_fn is not get_scan_fn(blk.scan_mode)


def _scan_fn_forward(blk, x):
    """MambaBlock.__call__ in the reference's op sequence
    (mamba_block.py:155-192), calling ``blk._scan_fn(x, delta, A, B, C, D)``
    at :187.  Used when a block's scan function was replaced; the conv +
    SiLU runs on the HIP conv kernel, the rest on torch ops."""
    din, ns, R = blk.d_inner, blk.d_state, blk.dt_rank
    xz = F.linear(x, blk.in_proj.weight)                                      # :165
    xb, z = xz[..., :din], xz[..., din:]                                       # :166-167
    conv_w = blk.conv1d.weight.reshape(1, din, blk.d_conv)
    xc = causal_conv_silu(xb.unsqueeze(2), conv_w, blk.conv1d.bias.unsqueeze(0)).squeeze(2)  # :170-171
    dbc = F.linear(xc, blk.x_proj.weight)                                      # :174
    dt, Bm, Cm = dbc[..., :R], dbc[..., R:R + ns], dbc[..., R + ns:]           # :175-177
    delta = F.softplus(F.linear(dt, blk.dt_proj.weight, blk.dt_proj.bias))     # :180-181
    A = -torch.exp(blk.A_log)                                                  # :184
    y = blk._scan_fn(xc, delta, A, Bm, Cm, blk.D)                              # :187
    y = y * F.silu(z)                                                          # :190
    return F.linear(y, blk.out_proj.weight)                                    # :191


def _per_direction_forward(blocks, h, tok):
    """Sum over directions of block k run on h in the scan order tok[k]
    (a gathered copy, as the reference builds, mamba_block.py:407-533), its
    output put back in token order.  Used when a block's scan function was
    replaced, so that each block's own ``__call__`` runs."""
    y = None
    for k, blk in enumerate(blocks):
        order = tok[k].long()
        out = blk(h[:, order])
        out = out[:, torch.argsort(order)]
        y = out if y is None else y + out
    return y


def _directional_forward(blocks, h, tok, scan_mode, stacks=None):
    """Run len(blocks) MambaBlocks on one (B, N, E) input, block k scanning
    in the order of tok[k], and return the sum of their outputs.  ``stacks``:
    the buffers of _direction_stacks whose leading slices hold the blocks'
    parameters (None: a single block, whose parameters are used as views)."""
    K = len(blocks)
    b0 = blocks[0]
    bsz, n, _ = h.shape
    din, ns, R = b0.d_inner, b0.d_state, b0.dt_rank
    if stacks is None:
        per = [ps[0].unsqueeze(0) for ps in _params_of([b0])]
    else:
        per = _DirectionParams.apply(len(stacks), *[buf[:K] for buf in stacks],
                                     *[p for ps in _params_of(blocks) for p in ps])
    W_in, conv_w, conv_b, W_x, W_dt, b_dt, A_log, Dv, W_out = per
    W_in = W_in.reshape(K * 2 * din, W_in.shape[-1])                          # (K*2D, E)
    xz = F.linear(h, W_in).view(bsz, n, K, 2 * din)                            # :165-167
    conv_w = conv_w.reshape(K, din, b0.d_conv)                                 # (K, Din, d_conv)
    # W_x (K, R+2N, Din), W_dt (K, Din, R), b_dt (K, Din), A_log (K, Din, N), Dv (K, Din)
    if tok is not None:
        tok = tok.to(h.device).contiguous()
    # the reference's "metal" mode is inference only (mamba_metal.py:230)
    detach = scan_mode == "metal"
    args = [t.float() for t in (xz, conv_w, conv_b, W_x, W_dt, b_dt, A_log, Dv)]
    if detach:
        args = [t.detach() for t in args]
    save = not detach and torch.is_grad_enabled() and any(t.requires_grad for t in args)
    y = _MambaCoreFn.apply(*args, tok, mode_chunk_len(scan_mode), save)       # :170-190
    # (K, E, Din) -> (E, K*Din): the out_proj of the concatenated directions
    # is their (atomic-free) sum
    W_out = W_out.permute(1, 0, 2).reshape(W_out.shape[1], K * din)
    return F.linear(y.reshape(bsz, n, K * din), W_out)                         # :191, :562-566
