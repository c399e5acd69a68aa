"""Torch CPU restatements of the reference -- TEST INFRASTRUCTURE ONLY.

See oracle/__init__.py: only tests/, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py`` use this module.

Two uses:

1. The CPU baseline.  ``scan_sequential`` and ``scan_chunked`` restate the
   reference's ``sequential`` and ``chunked`` scan modes op for op
   (materialised (B,L,D,N) discretisation, a Python loop over time, stack,
   skip term).  Their gradients come from torch autograd, as the reference's
   come from MLX autograd.  ``mlx`` is not installed, so these stand in for
   the reference's CPU run.

2. Module parity.  ``mamba_block``, ``direction_block`` and ``vision_mamba``
   are functional float64 restatements of mamba_block.py:155-192,
   :536-566 and vision_mamba.py:194-224.  They take the parameters of the
   product's modules by name and apply the reference's materialised
   permutations (reshape / transpose / flip), so that the product's
   index-remapped path is checked against the reference's formulation.
   They are pinned by closed forms in tests/test_oracle_blocks.py.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import ref_lib


# ---------------------------------------------------------------------------
# Scan modes
# ---------------------------------------------------------------------------

def scan_sequential(x, delta, A, B, C, D):
    """mamba_block.py:20-74 (the ``sequential`` mode)."""
    bsz, L, d = x.shape
    n = A.shape[1]
    delta_e = delta.unsqueeze(-1)                       # :51
    deltaA = torch.exp(delta_e * A[None, None])         # :52-53
    deltaBx = delta_e * B.unsqueeze(2) * x.unsqueeze(-1)  # :57-59
    h = x.new_zeros((bsz, d, n))                        # :62
    # per-step views taken with one unbind: the same arithmetic as indexing
    # [:, t], without autograd scattering every step's gradient into a
    # full-size zero tensor
    dA_t, dBx_t, C_t = deltaA.unbind(1), deltaBx.unbind(1), C.unbind(1)
    ys = []
    for t in range(L):                                  # :64
        h = dA_t[t] * h + dBx_t[t]                      # :65
        ys.append((h * C_t[t].unsqueeze(1)).sum(-1))    # :67
    y = torch.stack(ys, dim=1)                          # :70
    return y + x * D                                    # :73


def scan_chunked(x, delta, A, B, C, D, chunk_size=32):
    """mamba_fast.py:17-75 (the ``chunked`` mode)."""
    bsz, L, d = x.shape
    n = A.shape[1]
    delta_e = delta.unsqueeze(-1)
    deltaA = torch.exp(delta_e * A[None, None])          # :41-43
    deltaBx = delta_e * B.unsqueeze(2) * x.unsqueeze(-1)  # :45-47
    h = x.new_zeros((bsz, d, n))                          # :50
    parts = []
    for c0 in range(0, L, chunk_size):                    # :53
        c1 = min(c0 + chunk_size, L)
        dA_c = deltaA[:, c0:c1].unbind(1)
        dBx_c = deltaBx[:, c0:c1].unbind(1)
        C_c = C[:, c0:c1].unbind(1)
        ys = []
        for t in range(c1 - c0):                          # :64
            h = dA_c[t] * h + dBx_c[t]
            ys.append((h * C_c[t].unsqueeze(1)).sum(-1))
        parts.append(torch.stack(ys, dim=1))              # :70
    return torch.cat(parts, dim=1) + x * D                # :73-74


class _OracleScanFn(torch.autograd.Function):
    """The float64 C oracle (scan_ref.c, float64-input forms) as a torch op:
    forward mamba_block.py:45-74, VJP mamba_metal_fused.py:66-145,
    213-224.  Same function and gradients as ``scan_sequential`` (checked
    in tests/test_oracle_blocks.py), without a Python step per position, so
    the module restatements run at full sequence lengths in seconds."""

    @staticmethod
    def forward(ctx, x, delta, A, B, C, D):
        ctx.save_for_backward(x, delta, A, B, C, D)
        arrs = [t.detach().numpy() for t in (x, delta, A, B, C, D)]
        return torch.from_numpy(ref_lib.scan_fwd_f64(*arrs))

    @staticmethod
    def backward(ctx, gy):
        arrs = [t.detach().numpy() for t in ctx.saved_tensors]
        grads = ref_lib.scan_vjp_f64(*arrs, gy.detach().double().numpy())
        return tuple(torch.from_numpy(g) for g in grads)


def scan_oracle_c(x, delta, A, B, C, D):
    """float64 CPU scan with autograd through the C oracle; a drop-in for
    ``scan_sequential`` in the module restatements (float64 tensors)."""
    for t in (x, delta, A, B, C, D):
        if t.dtype != torch.float64 or t.device.type != "cpu":
            raise ValueError("scan_oracle_c takes float64 CPU tensors")
    return _OracleScanFn.apply(x, delta, A, B, C, D)


# ---------------------------------------------------------------------------
# Module restatements (float64 by default)
# ---------------------------------------------------------------------------

def _p(params, name, dtype):
    return params[name].detach().to(dtype).requires_grad_(params[name].requires_grad)


def mamba_block(params, prefix, x, d_state, d_conv, scan=scan_sequential):
    """MambaBlock.__call__, mamba_block.py:155-192, on a (B,L,E) sequence.

    ``params`` maps the product module's parameter names to tensors (already
    float64 leaves); ``prefix`` selects one block.
    """
    W_in = params[prefix + "in_proj.weight"]
    conv_w = params[prefix + "conv1d.weight"]     # (Din, 1, d_conv)
    conv_b = params[prefix + "conv1d.bias"]
    W_x = params[prefix + "x_proj.weight"]
    W_dt = params[prefix + "dt_proj.weight"]
    b_dt = params[prefix + "dt_proj.bias"]
    A_log = params[prefix + "A_log"]
    Dp = params[prefix + "D"]
    W_out = params[prefix + "out_proj.weight"]
    bsz, L, _ = x.shape
    d_inner = W_out.shape[1]
    dt_rank = W_dt.shape[1]
    xz = x @ W_in.T                                            # :165
    xb, z = xz[..., :d_inner], xz[..., d_inner:]               # :166-167
    # MLX Conv1d with padding d_conv-1 on both sides, then keep the first L
    # outputs (:129-132, :170): output t sees inputs t-d_conv+1 .. t, tap j
    # weighting input t - (d_conv - 1) + j (a cross-correlation), written
    # as a sum over the taps of the zero-padded sequence
    xp = F.pad(xb, (0, 0, d_conv - 1, 0))
    w = conv_w[:, 0, :]
    xc = conv_b + sum(xp[:, j:j + L] * w[:, j] for j in range(d_conv))
    xc = xc * torch.sigmoid(xc)                                # :171 SiLU
    dbc = xc @ W_x.T                                           # :174
    dt = dbc[..., :dt_rank]                                    # :175
    Bm = dbc[..., dt_rank:dt_rank + d_state]                   # :176
    Cm = dbc[..., dt_rank + d_state:]                          # :177
    delta = dt @ W_dt.T + b_dt                                 # :180
    delta = torch.log(1.0 + torch.exp(delta))                  # :181 softplus
    A = -torch.exp(A_log)                                      # :184
    y = scan(xc, delta, A, Bm, Cm, Dp)                         # :187
    y = y * (z * torch.sigmoid(z))                             # :190
    return y @ W_out.T                                         # :191


def layer_norm(params, prefix, x, eps=1e-5):
    """nn.LayerNorm with affine weight and bias (MLX default eps 1e-5)."""
    return F.layer_norm(x, (x.shape[-1],), params[prefix + "weight"],
                        params[prefix + "bias"], eps)


def _permute(h, grid_shape, axes_order):
    """_permute_2d_col_major / _permute_3d_axis / _permute_4d_axis,
    mamba_block.py:254-264, :277-290, :311-323."""
    bsz, n, e = h.shape
    nd = len(grid_shape)
    h = h.reshape(bsz, *grid_shape, e)
    perm = (0,) + tuple(a + 1 for a in axes_order) + (nd + 1,)
    return h.permute(perm).reshape(bsz, n, e)


def _unpermute(h, grid_shape, axes_order):
    """The matching inverses, mamba_block.py:267-274, :293-308, :326-338."""
    bsz, n, e = h.shape
    nd = len(grid_shape)
    permuted = tuple(grid_shape[a] for a in axes_order)
    h = h.reshape(bsz, *permuted, e)
    inv = [0] * nd
    for i, a in enumerate(axes_order):
        inv[a] = i
    perm = (0,) + tuple(a + 1 for a in inv) + (nd + 1,)
    return h.permute(perm).reshape(bsz, n, e)


_AXES = {
    2: [None],
    4: [None, (1, 0)],
    6: [None, (1, 0, 2), (2, 0, 1)],
    8: [None, (1, 0, 2, 3), (2, 0, 1, 3), (3, 0, 1, 2)],
}


def direction_block(params, prefix, x, num_directions, grid_shape, d_state,
                    d_conv, scan=scan_sequential):
    """MultiDirectionalMambaBlock.__call__ / _apply_direction,
    mamba_block.py:407-566 (materialised permutations and reverses)."""
    bsz, n, _ = x.shape
    h = layer_norm(params, prefix + "norm.", x)                # :548
    expected = 1
    for gdim in (grid_shape or (n,)):
        expected *= gdim
    K = num_directions
    if n != expected and K > 2:                                # :554-559
        y_f = mamba_block(params, prefix + "mamba_blocks.0.", h, d_state, d_conv, scan)
        y_b = mamba_block(params, prefix + "mamba_blocks.1.", h.flip(1), d_state, d_conv, scan).flip(1)
        return x + y_f + y_b
    y = None
    for k in range(K):                                         # :562-564
        pair, rev = divmod(k, 2)
        axes = _AXES[K][pair]
        seq = h if axes is None else _permute(h, grid_shape, axes)
        if rev:
            seq = seq.flip(1)
        out = mamba_block(params, f"{prefix}mamba_blocks.{k}.", seq, d_state, d_conv, scan)
        if rev:
            out = out.flip(1)
        if axes is not None:
            out = _unpermute(out, grid_shape, axes)
        y = out if y is None else y + out
    return x + y                                               # :566


def bidirectional_block(params, prefix, x, d_state, d_conv, scan=scan_sequential):
    """BidirectionalMambaBlock.__call__, mamba_block.py:226-237."""
    h = layer_norm(params, prefix + "norm.", x)
    y_f = mamba_block(params, prefix + "forward_mamba.", h, d_state, d_conv, scan)
    y_b = mamba_block(params, prefix + "backward_mamba.", h.flip(1), d_state, d_conv, scan).flip(1)
    return x + y_f + y_b


def vision_mamba(params, x, *, input_dim, patch_size, depth, grid_shape,
                 d_state, d_conv, temporal_patch_size=1, scan=scan_sequential,
                 patch_indices=None):
    """VisionMamba.__call__, vision_mamba.py:194-224, with PatchEmbed
    (vit.py:62-67), PatchEmbed3D (vit.py:87-92) and PatchEmbed4D
    (vision_mamba.py:65-94), all channel-last."""
    if x.ndim != 3:
        w = params["patch_embed.proj.weight"]
        b = params["patch_embed.proj.bias"]
        if input_dim == 2:
            out = F.conv2d(x.permute(0, 3, 1, 2), w, b, stride=patch_size)
            x = out.flatten(2).transpose(1, 2)
        elif input_dim == 3:
            out = F.conv3d(x.permute(0, 4, 1, 2, 3), w, b, stride=patch_size)
            x = out.flatten(2).transpose(1, 2)
        else:
            bsz, T, Dd, H, W, C = x.shape
            tp = temporal_patch_size
            if tp > 1:
                x = x.reshape(bsz, T // tp, tp, Dd, H, W, C).permute(0, 1, 3, 4, 5, 2, 6)
                x = x.reshape(bsz, T // tp, Dd, H, W, tp * C)
            t_out = T // tp
            x = x.reshape(bsz * t_out, Dd, H, W, -1)
            out = F.conv3d(x.permute(0, 4, 1, 2, 3), w, b, stride=patch_size)
            E = out.shape[1]
            out = out.permute(0, 2, 3, 4, 1)                    # channel-last
            x = out.reshape(bsz, -1, E)
    pos = params["pos_embed"]
    x = x + (pos[:, patch_indices, :] if patch_indices is not None else pos)
    K = {2: 4, 3: 6, 4: 8}[input_dim]
    for i in range(depth):
        x = direction_block(params, f"blocks.{i}.", x, K, grid_shape, d_state, d_conv, scan)
    return layer_norm(params, "norm.", x)


def params_from_module(module, dtype=torch.float64):
    """Detached float64 copies of a module's parameters, as grad leaves."""
    return {k: v.detach().to("cpu", dtype).clone().requires_grad_(True)
            for k, v in module.named_parameters()}


def softplus_inverse(dt):
    """dt_bias such that softplus(dt_bias) == dt."""
    return dt + torch.log(-torch.expm1(-dt))


def dt_rank_for(d_model):
    """mamba_block.py:136."""
    return math.ceil(d_model / 16)


# ---------------------------------------------------------------------------
# Error-magnitude companions (per-element bounds for the module parity tests)
# ---------------------------------------------------------------------------
#
# A first-order running error analysis of the restatements above, carried
# out alongside them.  Every tensor is a pair TC(v, m): its float64 value v
# and an error magnitude m >= |v| in units of 2^-24 (a float32 evaluation is
# expected within a small multiple of 2^-24 m of v).  Each operation with
# coefficients is an autograd Function over both channels:
#   forward   m_out = magnitudes of the terms forming the output with the
#             errors of the inputs (one magnitude times values per term);
#   backward  given the actual cotangent G and its magnitude MG, the value
#             channel gets the true gradient and the magnitude channel the
#             magnitude of that gradient's terms with the errors of their
#             factors (the cotangent's and the forward values').
# Shape-only operations (permute, flip, pad, slices, adds) act on both
# channels.  So one backward of <G, out.v> + <|G|, out.m> gives, for every
# parameter and input, the true gradient (value leaves) and its magnitude S
# (magnitude leaves: |p|, ones for A_log).  The value channel reproduces
# the restatements above (tests/test_oracle_blocks.py checks values and
# gradients against torch autograd of them).

class TC:
    """A (value, magnitude) pair."""

    def __init__(self, v, m):
        self.v, self.m = v, m

    def map(self, fn):
        return TC(fn(self.v), fn(self.m))

    def __add__(self, other):
        return TC(self.v + other.v, self.m + other.m)

    def __getitem__(self, idx):
        return TC(self.v[idx], self.m[idx])

    def flip(self, dim):
        return TC(self.v.flip(dim), self.m.flip(dim))


def _reduce_to(t, shape):
    return t.sum_to_size(shape) if t.shape != shape else t


class _LinFn(torch.autograd.Function):
    """Y = X W^T."""

    @staticmethod
    def forward(ctx, X, MX, W, MW):
        ctx.save_for_backward(X, MX, W, MW)
        return X @ W.T, MX @ MW.T

    @staticmethod
    def backward(ctx, G, MG):
        X, MX, W, MW = ctx.saved_tensors
        Xf, MXf = X.reshape(-1, X.shape[-1]), MX.reshape(-1, X.shape[-1])
        Gf, MGf = G.reshape(-1, G.shape[-1]), MG.reshape(-1, G.shape[-1])
        dW = Gf.T @ Xf
        MdW = MGf.T @ Xf.abs() + Gf.abs().T @ MXf
        return G @ W, MG @ MW, dW, MdW


class _MulFn(torch.autograd.Function):
    """a * b (broadcasting)."""

    @staticmethod
    def forward(ctx, a, Ma, b, Mb):
        ctx.save_for_backward(a, Ma, b, Mb)
        return a * b, Ma * b.abs() + a.abs() * Mb

    @staticmethod
    def backward(ctx, G, MG):
        a, Ma, b, Mb = ctx.saved_tensors
        da, db = G * b, G * a
        Mda = MG * b.abs() + G.abs() * Mb
        Mdb = MG * a.abs() + G.abs() * Ma
        return (_reduce_to(da, a.shape), _reduce_to(Mda, a.shape),
                _reduce_to(db, b.shape), _reduce_to(Mdb, b.shape))


def _pw_terms(kind, x):
    """(f, f', magnitude of the terms of f', a bound on |f''|)."""
    s = torch.sigmoid(x)
    if kind == "silu":
        return (x * s, s * (1 + x * (1 - s)), s * (1 + x.abs() * (1 - s)),
                s * (1 - s) * (2 + x.abs() * (1 - 2 * s).abs()))
    return F.softplus(x), s, s, s * (1 - s)   # softplus


class _PointwiseFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, Mx, kind):
        ctx.save_for_backward(x, Mx)
        ctx.kind = kind
        f, df, _, _ = _pw_terms(kind, x)
        return f, f.abs() + df.abs() * Mx

    @staticmethod
    def backward(ctx, G, MG):
        x, Mx = ctx.saved_tensors
        _, df, cdf, d2f = _pw_terms(ctx.kind, x)
        return G * df, MG * cdf + G.abs() * d2f * Mx, None


class _NegExpFn(torch.autograd.Function):
    """A = -exp(A_log) (mamba_block.py:184); the magnitude leaf is ones."""

    @staticmethod
    def forward(ctx, a_log, ones):
        A = -torch.exp(a_log)
        ctx.save_for_backward(A)
        return A, A.abs() * ones

    @staticmethod
    def backward(ctx, G, MG):
        (A,) = ctx.saved_tensors
        return G * A, (MG + G.abs()) * A.abs()


class _LayerNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, Mx, w, Mw, b, Mb, eps):
        mu = x.mean(-1, keepdim=True)
        var = ((x - mu) ** 2).mean(-1, keepdim=True)
        r = 1.0 / torch.sqrt(var + eps)
        xh = (x - mu) * r
        E = r * (Mx + Mx.mean(-1, keepdim=True) + xh.abs() * (xh.abs() * Mx).mean(-1, keepdim=True)) + xh.abs()
        # relative error of r (half that of var), in units of 2^-24
        rho = 1 + 0.5 * ((2 * (x - mu).abs() * (Mx + Mx.mean(-1, keepdim=True))).mean(-1, keepdim=True)
                         + var) / (var + eps)
        ctx.save_for_backward(xh, r, E, rho, w, Mw)
        return xh * w + b, E * w.abs() + Mw * xh.abs() + Mb

    @staticmethod
    def backward(ctx, G, MG):
        xh, r, E, rho, w, Mw = ctx.saved_tensors
        g = G * w
        Mg = MG * Mw
        mg, mgx = g.mean(-1, keepdim=True), (g * xh).mean(-1, keepdim=True)
        dx = r * (g - mg - xh * mgx)
        Mdx = (r * (Mg + Mg.mean(-1, keepdim=True) + xh.abs() * (Mg * xh.abs()).mean(-1, keepdim=True))
               + r * (E * mgx.abs() + xh.abs() * (g.abs() * E).mean(-1, keepdim=True)) + dx.abs() * rho)
        lead = tuple(range(G.dim() - 1))
        dw = (G * xh).sum(lead)
        Mdw = (MG * xh.abs() + G.abs() * E).sum(lead)
        return dx, Mdx, dw, Mdw, G.sum(lead), MG.sum(lead), None


class _ScanFn(torch.autograd.Function):
    """The scan (float64 C oracle) and its error magnitudes."""

    @staticmethod
    def forward(ctx, u, Mu, dl, Md, A, MA, B, MB, C, MC, D, MD):
        vals = [t.detach().numpy() for t in (u, dl, A, B, C, D)]
        mags = [t.detach().numpy() for t in (Mu, Md, MA, MB, MC, MD)]
        ctx.vals, ctx.mags = vals, mags
        return (torch.from_numpy(ref_lib.scan_fwd_f64(*vals)),
                torch.from_numpy(ref_lib.scan_mag_fwd(vals, mags)))

    @staticmethod
    def backward(ctx, G, MG):
        g = G.detach().double().numpy()
        grads = ref_lib.scan_vjp_f64(*ctx.vals, g)
        mags = ref_lib.scan_mag_vjp(ctx.vals, ctx.mags, g, MG.detach().double().numpy())
        out = []
        for a, m in zip(grads, mags):
            out += [torch.from_numpy(a), torch.from_numpy(m)]
        return tuple(out)


def tc_lin(x, W):
    return TC(*_LinFn.apply(x.v, x.m, W.v, W.m))


def tc_mul(a, b):
    return TC(*_MulFn.apply(a.v, a.m, b.v, b.m))


def tc_pointwise(kind, x):
    return TC(*_PointwiseFn.apply(x.v, x.m, kind))


def tc_params(params):
    """TC leaves for the module parameters: the value leaves are ``params``
    themselves (their .grad is the true gradient), the magnitude leaves |p|
    (ones for A_log; their .grad is the gradient's magnitude)."""
    out = {}
    for k, v in params.items():
        m = torch.ones_like(v) if k.endswith("A_log") else v.detach().abs()
        out[k] = TC(v, m.clone().requires_grad_(True))
    return out


def layer_norm_tc(P, prefix, x, eps=1e-5):
    w, b = P[prefix + "weight"], P[prefix + "bias"]
    return TC(*_LayerNormFn.apply(x.v, x.m, w.v, w.m, b.v, b.m, eps))


def mamba_block_tc(P, prefix, x, d_state, d_conv):
    """``mamba_block`` on TC pairs."""
    Q = {k[len(prefix):]: v for k, v in P.items() if k.startswith(prefix)}
    L = x.v.shape[1]
    d_inner = Q["out_proj.weight"].v.shape[1]
    dt_rank = Q["dt_proj.weight"].v.shape[1]
    xz = tc_lin(x, Q["in_proj.weight"])
    xb, z = xz[..., :d_inner], xz[..., d_inner:]
    xp = xb.map(lambda t: F.pad(t, (0, 0, d_conv - 1, 0)))
    cw = Q["conv1d.weight"]
    pre = Q["conv1d.bias"]
    for j in range(d_conv):
        pre = pre + tc_mul(xp[:, j:j + L], cw[:, 0, j])
    xc = tc_pointwise("silu", pre)
    dbc = tc_lin(xc, Q["x_proj.weight"])
    dt = dbc[..., :dt_rank]
    Bm = dbc[..., dt_rank:dt_rank + d_state]
    Cm = dbc[..., dt_rank + d_state:]
    delta = tc_pointwise("softplus", tc_lin(dt, Q["dt_proj.weight"]) + Q["dt_proj.bias"])
    A = TC(*_NegExpFn.apply(Q["A_log"].v, Q["A_log"].m))
    Dp = Q["D"]
    y = TC(*_ScanFn.apply(xc.v, xc.m, delta.v, delta.m, A.v, A.m, Bm.v, Bm.m, Cm.v, Cm.m,
                          Dp.v, Dp.m))
    y = tc_mul(y, tc_pointwise("silu", z))
    return tc_lin(y, Q["out_proj.weight"])


def residual_block_tc(P, prefix, x, d_state, d_conv):
    """ResidualMambaBlock: x + mamba(norm(x)) (mamba_block.py:195-205)."""
    return x + mamba_block_tc(P, prefix + "mamba.", layer_norm_tc(P, prefix + "norm.", x),
                              d_state, d_conv)


def bidirectional_block_tc(P, prefix, x, d_state, d_conv):
    h = layer_norm_tc(P, prefix + "norm.", x)
    yf = mamba_block_tc(P, prefix + "forward_mamba.", h, d_state, d_conv)
    yb = mamba_block_tc(P, prefix + "backward_mamba.", h.flip(1), d_state, d_conv)
    return x + yf + yb.flip(1)


def direction_block_tc(P, prefix, x, num_directions, grid_shape, d_state, d_conv):
    n = x.v.shape[1]
    h = layer_norm_tc(P, prefix + "norm.", x)
    expected = 1
    for gdim in (grid_shape or (n,)):
        expected *= gdim
    K = num_directions
    if n != expected and K > 2:
        yf = mamba_block_tc(P, prefix + "mamba_blocks.0.", h, d_state, d_conv)
        yb = mamba_block_tc(P, prefix + "mamba_blocks.1.", h.flip(1), d_state, d_conv)
        return x + yf + yb.flip(1)
    y = x
    for k in range(K):
        pair, rev = divmod(k, 2)
        axes = _AXES[K][pair]
        seq = h if axes is None else h.map(lambda t: _permute(t, grid_shape, axes))
        if rev:
            seq = seq.flip(1)
        out = mamba_block_tc(P, f"{prefix}mamba_blocks.{k}.", seq, d_state, d_conv)
        if rev:
            out = out.flip(1)
        if axes is not None:
            out = out.map(lambda t: _unpermute(t, grid_shape, axes))
        y = y + out
    return y


def vision_mamba_tc(P, x, *, input_dim, patch_size, depth, grid_shape, d_state, d_conv,
                    temporal_patch_size=1, patch_indices=None):
    """``vision_mamba`` on TC pairs (the patch embedding as a linear map of
    the flattened patches)."""
    if x.v.ndim != 3:
        W = P["patch_embed.proj.weight"]
        E = W.v.shape[0]
        W2 = W.map(lambda t: t.reshape(E, -1))
        p = patch_size
        if input_dim == 2:
            bsz, H, Wd, C = x.v.shape

            def patches(t):
                t = t.reshape(bsz, H // p, p, Wd // p, p, C).permute(0, 1, 3, 5, 2, 4)
                return t.reshape(bsz, (H // p) * (Wd // p), C * p * p)
        else:
            if input_dim == 3:
                bsz, Dd, H, Wd, C = x.v.shape
                fold = lambda t: t                                        # noqa: E731
            else:
                bsz0, T, Dd, H, Wd, C0 = x.v.shape
                tp = temporal_patch_size

                def fold(t):
                    if tp > 1:
                        t = t.reshape(bsz0, T // tp, tp, Dd, H, Wd, C0).permute(0, 1, 3, 4, 5, 2, 6)
                        t = t.reshape(bsz0, T // tp, Dd, H, Wd, tp * C0)
                    return t.reshape(bsz0 * (T // tp), Dd, H, Wd, -1)
                C = C0 * tp
                bsz = bsz0 * (T // tp)

            def patches(t):
                t = fold(t).reshape(bsz, Dd // p, p, H // p, p, Wd // p, p, C)
                t = t.permute(0, 1, 3, 5, 7, 2, 4, 6)
                return t.reshape(bsz, -1, C * p * p * p)
        x = tc_lin(x.map(patches), W2) + P["patch_embed.proj.bias"]
        if input_dim == 4:
            x = x.map(lambda t: t.reshape(bsz0, -1, E))
    pos = P["pos_embed"]
    if patch_indices is not None:
        pos = pos[:, patch_indices, :]
    x = x + pos
    K = {2: 4, 3: 6, 4: 8}[input_dim]
    for i in range(depth):
        x = direction_block_tc(P, f"blocks.{i}.", x, K, grid_shape, d_state, d_conv)
    return layer_norm_tc(P, "norm.", x)


def run_tc(fn, params, x, G):
    """Runs a ``*_tc`` restatement on float64 parameter leaves ``params``
    and input x with output cotangent G.  Returns (output, grads, S): the
    output value, {"input grad", "grad <param>"} true gradients, and the
    magnitudes {"output", "input grad", "grad <param>"}."""
    P = tc_params(params)
    xv = x.detach().double().clone().requires_grad_(True)
    xm = xv.detach().abs().requires_grad_(True)
    out = fn(P, TC(xv, xm))
    G = G.detach().double()
    ((G * out.v).sum() + (G.abs() * out.m).sum()).backward()
    grads = {"input grad": xv.grad}
    S = {"output": out.m.detach(), "input grad": xm.grad}
    for k, t in P.items():
        if t.m.grad is not None:
            grads[f"grad {k}"] = t.v.grad
            S[f"grad {k}"] = t.m.grad
    return out.v.detach(), grads, S
