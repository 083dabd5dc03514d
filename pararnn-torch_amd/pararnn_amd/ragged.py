"""Packed ragged batches (``cu_seqlens``) and paged ``h0`` (``block_table``).

The reference packs S sequences into one stream ``(1, N, ...)`` with
FlashAttention-style offsets ``cu_seqlens`` ``(S+1,)`` and drops the carry at
each sequence head (J = 0 there, ``h0[s]`` as the previous state;
``layout.py:93-138``, ``solvers/scan.py:206-216``).  Sequences never interact,
so this build runs them as a padded rectangular batch ``(S, T_max, ...)``
through the same fused kernels: every sequence starts from its own ``h0``
exactly as at a head, positions past a sequence's end are computed and
discarded (they come after it in time, so they cannot reach it), and the
result is gathered back into the packed order.  Padding and gathering are
differentiable index operations, so the eq. 2.6 backward runs unchanged (the
upstream gradient at discarded positions is zero, so nothing flows from them).
"""

from __future__ import annotations

import torch
from torch import Tensor


def validate_cu_seqlens(cu_seqlens: Tensor, time: int) -> Tensor:
    """``(S+1,)`` exclusive prefix with ``[0] = 0``, last = ``time``, strictly increasing
    (layout.py:93-104)."""
    if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
        raise ValueError(f"cu_seqlens must be (S+1,), got {tuple(cu_seqlens.shape)}")
    cs = cu_seqlens.to(dtype=torch.long)
    if int(cs[0]) != 0:
        raise ValueError(f"cu_seqlens[0] must be 0, got {int(cs[0])}")
    if int(cs[-1]) != int(time):
        raise ValueError(f"cu_seqlens[-1] must equal time={time}, got {int(cs[-1])}")
    if torch.any(cs[1:] <= cs[:-1]):
        raise ValueError("cu_seqlens must be strictly increasing")
    return cs


def segment_start_flags(cu_seqlens: Tensor, time: int, *, batch: int = 1) -> Tensor:
    """Bool ``(batch, time)``: True at the first token of each packed sequence."""
    cs = validate_cu_seqlens(cu_seqlens, time)
    flags = torch.zeros(batch, time, dtype=torch.bool, device=cs.device)
    flags[:, cs[:-1]] = True
    return flags


def prepend_state_ragged(states: Tensor, h0: Tensor | None, cu_seqlens: Tensor) -> Tensor:
    """Previous state at every packed position: ``h0[s]`` (or zeros) at the head of
    sequence s, else the state one step back (layout.py:115-138)."""
    if states.shape[0] != 1:
        raise ValueError(f"ragged prepend needs packed batch 1, got batch={states.shape[0]}")
    cs = validate_cu_seqlens(cu_seqlens, states.shape[1]).to(states.device)
    out = states.new_empty(states.shape)
    out[:, 1:] = states[:, :-1]
    starts = cs[:-1]
    if h0 is None:
        out[:, starts] = 0
    else:
        if h0.shape[0] != cs.numel() - 1:
            raise ValueError(f"h0 batch {h0.shape[0]} != n_seq {cs.numel() - 1}")
        out[0, starts] = h0.to(states.dtype)
    return out


class Padding:
    """Index maps between a packed stream ``(1, N, ...)`` and ``(S, T_max, ...)``."""

    def __init__(self, cs: Tensor, device: torch.device) -> None:
        cs = cs.to(device)
        lengths = cs[1:] - cs[:-1]
        self.n_seq = int(lengths.numel())
        self.t_max = int(lengths.max())
        self.n = int(cs[-1])
        steps = torch.arange(self.t_max, device=device)
        self.mask = steps[None, :] < lengths[:, None]  # (S, T_max)
        self.index = (cs[:-1, None] + steps[None, :]).clamp(max=self.n - 1)

    def pad(self, packed: Tensor) -> Tensor:
        """``(1, N, ...)`` -> ``(S, T_max, ...)`` with zeros past each sequence's end."""
        g = packed[0][self.index]
        m = self.mask.reshape(*self.mask.shape, *([1] * (g.dim() - 2)))
        return torch.where(m, g, torch.zeros((), dtype=g.dtype, device=g.device))

    def unpad(self, padded: Tensor) -> Tensor:
        """``(S, T_max, ...)`` -> ``(1, N, ...)`` in packed order."""
        return padded[self.mask].unsqueeze(0)


def gather_h0(h0: Tensor | None, block_table: Tensor | None, n_rows: int,
              tail: tuple[int, ...]) -> Tensor | None:
    """Dense ``h0`` of ``n_rows`` rows: the pool rows ``block_table`` names, or ``h0``
    itself (kernels/_fused_common.py:106-139, kernels/fused_newton.py:344-345)."""
    if block_table is None:
        return h0
    if h0 is None:
        raise ValueError("block_table needs h0 as a pool (C, ...)")
    bt = block_table.to(device=h0.device, dtype=torch.long)
    if bt.dim() != 1:
        raise ValueError(f"block_table must be 1-D (B,), got {tuple(bt.shape)}")
    if int(bt.numel()) != n_rows:
        raise ValueError(f"block_table B={int(bt.numel())} != {n_rows}")
    if tuple(h0.shape[1:]) != tuple(tail):
        raise ValueError(f"pool h0 tail {tuple(h0.shape[1:])} != {tuple(tail)}")
    if int(h0.shape[0]) < 1:
        raise ValueError("pool h0 is empty")
    if bt.numel():
        mn, mx = int(bt.min()), int(bt.max())
        if mn < 0 or mx >= int(h0.shape[0]):
            raise ValueError(f"block_table slots [{mn}, {mx}] outside pool capacity "
                             f"{int(h0.shape[0])}")
    return h0.index_select(0, bt)
