"""Float64 CPU restatement of the reference's selective scan -- TEST INFRASTRUCTURE ONLY.

This module is the oracle: the checker that the HIP path is compared against.
Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import it.  Nothing in the product package uses it.

Every function cites the reference lines it restates (paths are relative to
the reference repository root).  All arithmetic is float64 numpy.

Pinning (each function is checked by something other than a retyped formula):

* ``scan_fwd``        closed forms (L=1, A=0 -> cumsum, constant decay ->
                      ``scipy.signal.lfilter``, delta=0, B=0, C=0), linearity
                      in u, brute-force scalar loop; tests/test_oracle.py.
* ``scan_vjp``        ``torch.autograd`` through an independent torch float64
                      forward, ``torch.autograd.gradcheck`` finite differences,
                      closed forms dD = sum(g*u) and the delta=0 dδ formula.
* ``scan_fwd_chunked`` equals ``scan_fwd`` for chunk=1, chunk=L and any chunk.
* ``combine``          associativity, checked numerically.
* ``fused_fwd`` / ``fused_vjp``  (the block's softplus prologue and gated
                      epilogue around the scan) torch float64 autograd through
                      ``F.softplus`` / ``F.silu`` and the independent torch
                      scan restatement; tests/test_oracle.py.
* ``direction_axis_order`` / ``seq_to_token``  the materialised torch
                      reshape / permute / flip of the reference's helpers and
                      a hand-derived K=6 case; tests/test_oracle.py.

The other oracle pieces are pinned in the same way:

* scan_ref.c ``oracle_scan_fwd`` / ``oracle_scan_vjp``: equal to this module
  (tests/test_oracle.py::test_c_oracle_matches_numpy).
* scan_ref.c ``oracle_ddelta_scale`` (the cancellation scale S that widens
  the ddelta bound): S >= |ddelta| everywhere, S = |ddelta| exactly on
  inputs whose terms share one sign (both terms exercised), the delta = 0
  closed form over a reverse cumsum, and homogeneity in g and u.
* scan_ref.c ``oracle_dA_scale`` (the cancellation scale of dA, the sum of
  the magnitudes of its lam delta e h terms): S >= |dA| everywhere,
  S = dA exactly when every term is positive, a scalar brute-force loop on a
  tiny case, S = 0 at L = 1, and homogeneity in g and u.
* torch_ref ``scan_sequential`` / ``scan_chunked``: autograd and
  ``gradcheck`` (tests/test_oracle.py); ``mamba_block``, ``layer_norm``,
  ``direction_block``, ``bidirectional_block``, ``vision_mamba``: closed
  forms from ``np.convolve`` / ``np.cumsum`` at unit decay, a hand-written
  two-token scan with decay, a textbook LayerNorm, numpy-built scan orders
  and a brute-force patch embedding, each shown sensitive to the plausible
  mistakes (tests/test_oracle_blocks.py).

No golden vectors exist in the reference (it has no tests).  The fixtures
under tests/golden/ are written from this oracle (and scan_ref.c) by
tests/golden/make_golden.py after the checks above pass; tests/test_golden.py
checks that the oracle still reproduces them.
"""

from __future__ import annotations

import numpy as np


def _f64(*xs):
    return [np.asarray(x, dtype=np.float64) for x in xs]


def discretize(u, delta, A, B):
    """Materialised discretisation, mamba_block.py:51-59.

    Returns (dA, dBu), both (B, L, D, N):
        dA  = exp(delta[..., None] * A)            (mamba_block.py:51-53)
        dBu = delta[..., None] * B[:, :, None] * u[..., None]   (:57-59)
    """
    u, delta, A, B = _f64(u, delta, A, B)
    dA = np.exp(delta[..., None] * A[None, None, :, :])
    dBu = delta[..., None] * B[:, :, None, :] * u[..., None]
    return dA, dBu


def scan_fwd(u, delta, A, B, C, D, return_states=False):
    """Sequential selective scan, mamba_block.py:20-74.

    u, delta: (B, L, D); A: (D, N); B, C: (B, L, N); D: (D,).
    h_{-1} = 0; h_t = dA_t * h_{t-1} + dBu_t  (:62-65)
    y_t = sum_n h_t[n] * C_t[n]               (:67)
    y += u * D                                 (:73)
    """
    u, delta, A, B, C, D = _f64(u, delta, A, B, C, D)
    bsz, L, d = u.shape
    n = A.shape[1]
    dA, dBu = discretize(u, delta, A, B)
    h = np.zeros((bsz, d, n))
    ys = np.empty((bsz, L, d))
    hs = np.empty((bsz, L, d, n)) if return_states else None
    for t in range(L):
        h = dA[:, t] * h + dBu[:, t]
        ys[:, t] = np.einsum("bdn,bn->bd", h, C[:, t])
        if return_states:
            hs[:, t] = h
    y = ys + u * D
    if return_states:
        return y, hs
    return y


def scan_fwd_chunked(u, delta, A, B, C, D, chunk_size=32):
    """The ``chunked`` scan_mode, mamba_fast.py:17-75.

    Same per-step arithmetic as ``scan_fwd`` run inside an outer loop over
    chunks of ``chunk_size`` (:53-67); the carry h crosses chunk boundaries.
    """
    u, delta, A, B, C, D = _f64(u, delta, A, B, C, D)
    bsz, L, d = u.shape
    n = A.shape[1]
    dA, dBu = discretize(u, delta, A, B)
    h = np.zeros((bsz, d, n))
    parts = []
    for c0 in range(0, L, chunk_size):
        c1 = min(c0 + chunk_size, L)
        ys = []
        for t in range(c0, c1):
            h = dA[:, t] * h + dBu[:, t]
            ys.append(np.einsum("bdn,bn->bd", h, C[:, t]))
        parts.append(np.stack(ys, axis=1))
    return np.concatenate(parts, axis=1) + u * D


def combine(p1, p2):
    """Associative operator of the linear recurrence, mamba_fast.py:85-86.

    (a1, b1) (+) (a2, b2) = (a2 * a1, a2 * b1 + b2): applying step 1 then
    step 2 to a state h gives a2*(a1*h + b1) + b2.
    """
    a1, b1 = p1
    a2, b2 = p2
    return a2 * a1, a2 * b1 + b2


def scan_fwd_two_pass(u, delta, A, B, C, D, chunk_len):
    """Two-pass chunked scan (the carry step the reference left as TODO at
    mamba_metal_chunked.py:268-272), written with ``combine``.

    Pass 1 reduces each chunk to its aggregate (prod dA, local end state from
    h=0); pass 2 folds the aggregates left to right into each chunk's
    carry-in; pass 3 rescans every chunk from its carry-in.
    """
    u, delta, A, B, C, D = _f64(u, delta, A, B, C, D)
    bsz, L, d = u.shape
    n = A.shape[1]
    dA, dBu = discretize(u, delta, A, B)
    starts = list(range(0, L, chunk_len))
    aggs = []
    for c0 in starts:
        agg = (np.ones((bsz, d, n)), np.zeros((bsz, d, n)))
        for t in range(c0, min(c0 + chunk_len, L)):
            agg = combine(agg, (dA[:, t], dBu[:, t]))
        aggs.append(agg)
    carry = np.zeros((bsz, d, n))
    y = np.empty((bsz, L, d))
    for ci, c0 in enumerate(starts):
        h = carry
        for t in range(c0, min(c0 + chunk_len, L)):
            h = dA[:, t] * h + dBu[:, t]
            y[:, t] = np.einsum("bdn,bn->bd", h, C[:, t])
        a, b = aggs[ci]
        carry = a * carry + b
    return y + u * D


def scan_vjp(u, delta, A, B, C, D, g):
    """Reverse-scan VJP of ``scan_fwd``; restates the adjoint recurrence of
    mamba_metal_fused.py:66-145 and the reductions at :213-224.

    lam accumulates C_t * g_t (:92-94), the per-step grads read lam and the
    previous state h_{t-1} (:105-133), then lam is scaled by dA_t (:136).

    Returns (du, ddelta, dA, dB, dC, dD) shaped like (u, delta, A, B, C, D).
    """
    u, delta, A, B, C, D, g = _f64(u, delta, A, B, C, D, g)
    bsz, L, d = u.shape
    n = A.shape[1]
    dA_t, _ = discretize(u, delta, A, B)
    _, hs = scan_fwd(u, delta, A, B, C, D, return_states=True)
    lam = np.zeros((bsz, d, n))
    du = np.empty((bsz, L, d))
    ddelta = np.empty((bsz, L, d))
    dA = np.zeros((d, n))
    dB = np.empty((bsz, L, n))
    dC = np.empty((bsz, L, n))
    for t in range(L - 1, -1, -1):
        lam = lam + C[:, t, None, :] * g[:, t, :, None]              # :92-94
        h_prev = hs[:, t - 1] if t > 0 else np.zeros((bsz, d, n))    # :105-112
        e = dA_t[:, t]
        ddelta[:, t] = np.sum(lam * (h_prev * A[None] * e
                                     + B[:, t, None, :] * u[:, t, :, None]), axis=-1)  # :116-117
        dA += np.sum(lam * h_prev * delta[:, t, :, None] * e, axis=0)   # :122, :218
        dB[:, t] = np.sum(lam * (delta[:, t] * u[:, t])[..., None], axis=1)  # :130, :221
        du[:, t] = D * g[:, t] + np.sum(lam * delta[:, t, :, None] * B[:, t, None, :], axis=-1)  # :87,:133
        dC[:, t] = np.sum(g[:, t, :, None] * hs[:, t], axis=1)        # :224
        lam = lam * e                                                 # :136
    dD = np.sum(g * u, axis=(0, 1))                                   # :89, :214
    return du, ddelta, dA, dB, dC, dD


# ---------------------------------------------------------------------------
# Block prologue / epilogue around the scan (the fused form)
# ---------------------------------------------------------------------------

def softplus(x):
    """softplus as the block applies it to dt_proj's output
    (mamba_block.py:181), with torch's linear branch above x = 20."""
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 20.0, x, np.logaddexp(0.0, x))


def sigmoid(x):
    """1 / (1 + e^-x), evaluated without overflow for either sign of x."""
    x = np.asarray(x, dtype=np.float64)
    e = np.exp(-np.abs(x))
    return np.where(x >= 0, 1.0 / (1.0 + e), e / (1.0 + e))


def fused_fwd(u, delta_raw, bias, A, B, C, D, z):
    """mamba_block.py:180-190 around the scan:
        delta = softplus(delta_raw + bias)   (:180-181, bias = dt_proj.bias)
        y_raw = scan(u, delta, A, B, C, D)   (:187)
        y     = y_raw * silu(z)              (:190)
    bias may be None (zero), z None (no gate).  Returns (y, y_raw, delta)."""
    delta_raw = np.asarray(delta_raw, dtype=np.float64)
    x = delta_raw + (0.0 if bias is None else np.asarray(bias, dtype=np.float64))
    delta = softplus(x)
    y_raw = scan_fwd(u, delta, A, B, C, D)
    if z is None:
        return y_raw, y_raw, delta
    z = np.asarray(z, dtype=np.float64)
    return y_raw * z * sigmoid(z), y_raw, delta


def fused_vjp(u, delta_raw, bias, A, B, C, D, z, g):
    """VJP of ``fused_fwd`` for upstream g (the gradient of the gated y):
    the gate's product and silu derivatives, ``scan_vjp`` on
    g * silu(z), and softplus' derivative (sigmoid; 1 above the threshold).
    Returns (du, ddelta_raw, dbias, dA, dB, dC, dD, dz); dbias sums over
    (b, t), dz is None without a gate."""
    delta_raw, g = _f64(delta_raw, g)
    x = delta_raw + (0.0 if bias is None else np.asarray(bias, dtype=np.float64))
    delta = softplus(x)
    if z is None:
        gs, dz = g, None
    else:
        z = np.asarray(z, dtype=np.float64)
        s = sigmoid(z)
        y_raw = scan_fwd(u, delta, A, B, C, D)
        gs = g * z * s
        dz = g * y_raw * s * (1.0 + z * (1.0 - s))
    du, dd, dA, dB, dC, dD = scan_vjp(u, delta, A, B, C, D, gs)
    ddelta_raw = dd * np.where(x > 20.0, 1.0, sigmoid(x))
    dbias = ddelta_raw.sum(axis=(0, 1))
    return du, ddelta_raw, dbias, dA, dB, dC, dD, dz


# ---------------------------------------------------------------------------
# Direction remaps (index form of the reference's permute/reverse helpers)
# ---------------------------------------------------------------------------

def direction_axis_order(num_directions, k):
    """Axis order and reverse flag of direction k, mamba_block.py:407-533.

    K=2: identity, reversed identity (:443-448).
    K=4: row-major, reversed, column-major (1,0), reversed (:450-473).
    K=6: (0,1,2), (1,0,2), (2,0,1), each then reversed (:475-504).
    K=8: (0,1,2,3), (1,0,2,3), (2,0,1,3), (3,0,1,2), each reversed (:506-533).
    Returns (axes_order or None for identity, reverse).
    """
    pair, rev = divmod(k, 2)
    rev = bool(rev)
    if num_directions == 2:
        return None, rev
    if num_directions == 4:
        return [None, (1, 0)][pair], rev
    if num_directions == 6:
        return [(0, 1, 2), (1, 0, 2), (2, 0, 1)][pair], rev
    if num_directions == 8:
        return [(0, 1, 2, 3), (1, 0, 2, 3), (2, 0, 1, 3), (3, 0, 1, 2)][pair], rev
    raise ValueError(num_directions)


def seq_to_token(n_tokens, grid_shape, axes_order, reverse):
    """Token read at each scan position, by materialising the reference's
    permutation on an index array (mamba_block.py:254-338 use reshape +
    transpose; the reverse slice ``[:, ::-1]`` is applied after the permute,
    :458-462, :466-472).
    """
    n = int(n_tokens)
    if axes_order is None:
        idx = np.arange(n)
    else:
        idx = np.arange(n).reshape(grid_shape).transpose(axes_order).reshape(-1)
    if reverse:
        idx = idx[::-1]
    return np.ascontiguousarray(idx)
