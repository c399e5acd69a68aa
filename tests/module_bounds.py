"""Per-element error bounds for the module parity tests.

For a module output or gradient with float64 reference ``ref`` the bound is

    |got - ref| <= 1e-5 + 1e-4 |ref| + min(C_MOD * 2^-24 * S, 1e-4 * max|ref|)

per element, where S is the error magnitude from the oracle's running error analysis
of the restatement (oracle/torch_ref.py ``*_tc``): for every element, the
magnitudes of the terms that form it, each with the errors of its factors
propagated from the inputs and parameters through every layer, forward and
backward (S >= |ref|; a float32 evaluation is expected within a small
multiple of 2^-24 S).  S is a worst-case sum: where it exceeds
1e-4 * max|ref| / C_MOD, the per-tensor term of the earlier bar applies
instead, so the bound is never looser than that bar.

Evidence for C_MOD: the reference's own algorithm evaluated in float32
(oracle/torch_ref.py in float32, the reference's precision) stays within
about 1.1 * 2^-24 * S (tests/test_oracle_blocks.py asserts 2).
"""

import torch

from oracle import torch_ref

C_MOD = 8
EPS = 2.0 ** -24


def magnitudes(tc_fn, params, x, G):
    """Value and error magnitudes of a module restatement on TC pairs
    (oracle/torch_ref.py ``*_tc``) for input x and output cotangent G:
    (output value, {"output", "input grad", "grad <param>"} -> S)."""
    leaves = {k: v.detach().clone().requires_grad_(True) for k, v in params.items()}
    val, _, S = torch_ref.run_tc(tc_fn, leaves, x, G)
    return val, S


def check(name, got, ref, S=None, c=C_MOD, log=None, cap=True):
    """Asserts the bound above (S None: the per-tensor bar alone; cap False:
    without the min with the per-tensor term) and returns the worst
    err / (2^-24 S)."""
    got = got.detach().double().cpu()
    ref = ref.detach().double()
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert torch.isfinite(got).all(), name
    scale = float(ref.abs().max()) if ref.numel() else 0.0
    err = (got - ref).abs()
    if S is None:
        bound = 1e-4 * scale + 1e-4 * ref.abs()
        worst = None
    else:
        S = S.detach().double()
        term = c * EPS * S
        if cap:
            term = torch.minimum(term, torch.full_like(S, 1e-4 * scale))
        bound = 1e-5 + 1e-4 * ref.abs() + term
        worst = float((err / (EPS * S).clamp_min(1e-300)).max()) if err.numel() else 0.0
        if log is not None:
            log.append((name, worst))
    if err.numel() and bool((err > bound).any()):
        i = int(torch.argmax(err - bound))
        raise AssertionError(f"{name}: max err {float(err.max()):.3e} (scale {scale:.3e}); worst flat "
                             f"index {i}: got {float(got.flatten()[i])}, ref {float(ref.flatten()[i])}, "
                             f"bound {float(bound.flatten()[i]):.3e}")
    return worst
