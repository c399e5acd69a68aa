"""Scan-order index tables for the multi-directional blocks.

The reference reorders the token sequence with materialised reshape /
transpose / reverse copies before each directional MambaBlock and undoes
them afterwards (mamba_block.py:254-338, :407-533).  Here each direction is
an int32 table ``seq_to_tok[k, s]`` = the token read at scan position s;
the scan kernel and the causal conv read and write through it, so no
permuted copy of the activations is made.

Direction semantics follow the reference exactly (including its labels):
  K=2: identity, reversed                                (:443-448)
  K=4: row-major, reversed, column-major (1,0), reversed (:450-473)
  K=6: axis orders (0,1,2), (1,0,2), (2,0,1), each then reversed (:475-504)
  K=8: axis orders (0,1,2,3), (1,0,2,3), (2,0,1,3), (3,0,1,2), each reversed
       (:506-533)
The reverse is applied after the permutation (scan position s reads token
perm(N-1-s), :458-472).
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import torch

_AXES = {
    2: [None],
    4: [None, (1, 0)],
    6: [None, (1, 0, 2), (2, 0, 1)],
    8: [None, (1, 0, 2, 3), (2, 0, 1, 3), (3, 0, 1, 2)],
}


def axis_order(num_directions: int, k: int) -> Tuple[Optional[Tuple[int, ...]], bool]:
    """(axes order or None for the identity, reverse flag) of direction k."""
    if num_directions not in _AXES:
        raise ValueError(f"num_directions must be 2, 4, 6 or 8; got {num_directions}")
    pair, rev = divmod(k, 2)
    return _AXES[num_directions][pair], bool(rev)


def seq_to_tok_table(num_directions: int, n_tokens: int,
                     grid_shape: Optional[Sequence[int]] = None) -> torch.Tensor:
    """(K, n_tokens) int32 CPU table.  With a grid, n_tokens must equal its
    size; without one only the identity / reversed orders exist (K=2)."""
    K = num_directions
    rows = []
    for k in range(K):
        axes, rev = axis_order(K, k)
        if axes is None:
            idx = torch.arange(n_tokens)
        else:
            if grid_shape is None or math.prod(grid_shape) != n_tokens:
                raise ValueError(f"direction {k} of K={K} needs a grid with {n_tokens} cells")
            idx = torch.arange(n_tokens).reshape(*grid_shape).permute(*axes).reshape(-1)
        if rev:
            idx = idx.flip(0)
        rows.append(idx)
    table = torch.stack(rows).to(torch.int32)
    # every row must be a permutation of the tokens
    check = torch.sort(table.long(), dim=1).values
    if not torch.equal(check, torch.arange(n_tokens).expand(K, n_tokens)):
        raise AssertionError("direction table is not a permutation")
    return table.contiguous()


def inverse_table(table: torch.Tensor) -> torch.Tensor:
    """tok_to_seq[k, n] = the scan position of token n in direction k."""
    inv = torch.empty_like(table)
    pos = torch.arange(table.shape[1], dtype=table.dtype, device=table.device)
    inv.scatter_(1, table.long(), pos.expand_as(table).contiguous())
    return inv
