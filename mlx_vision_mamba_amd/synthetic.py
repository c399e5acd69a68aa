"""Seeded synthetic selective-scan inputs (the benchmark workloads' recipe),
used by bench.py and the tests.

Recipe (generated in this order on a CPU torch.Generator):
u ~ N(0,1) (B,L,D); delta = softplus(0.5*N(0,1) - 4.6) (B,L,D), i.e. dt in
about [1e-3, 1e-1]; A[d,n] = -(n+1) (S4D-real); B, C ~ N(0,1) (B,L,N);
D = 1; upstream gradient g ~ N(0,1) (B,L,D).
"""

import torch


def make(bsz, L, D, N, seed=0, dtype=torch.float32, a_mode="s4d"):
    gen = torch.Generator().manual_seed(seed)
    u = torch.randn(bsz, L, D, generator=gen)
    delta = torch.nn.functional.softplus(torch.randn(bsz, L, D, generator=gen) * 0.5 - 4.6)
    if a_mode == "s4d":
        A = -torch.arange(1, N + 1, dtype=torch.float32).repeat(D, 1)
    else:  # random negative decay rates, not tied to the state index
        A = -torch.exp(torch.randn(D, N, generator=gen))
    Bm = torch.randn(bsz, L, N, generator=gen)
    Cm = torch.randn(bsz, L, N, generator=gen)
    Dv = torch.ones(D)
    g = torch.randn(bsz, L, D, generator=gen)
    if dtype != torch.float32:
        u, Bm, Cm, g = (t.to(dtype) for t in (u, Bm, Cm, g))
    return u, delta, A, Bm, Cm, Dv, g
