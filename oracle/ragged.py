"""Packed ragged batches (``cu_seqlens``) for the oracle (test infrastructure only).

The reference solves a packed stream ``(1, N, ...)`` with the carry dropped at
every sequence head (J = 0 there) and ``h0[s]`` as the previous state of
sequence s (``layout.py:93-138``, ``solvers/scan.py:206-216``); its Picard
frozen-gate scans restart per segment (``solvers/slstm_picard.py:51-140``).
With the carry dropped, the sequences are independent, so the same iterate is
each sequence solved on its own with the same K and P (P resolved from the
packed length N, as ``newton_apply`` resolves it before the solve), then
concatenated; the reference's segmented fp32 scans round in a different order.
"""

from __future__ import annotations

import torch
from torch import Tensor

from oracle.gru_head import GRUHeadParams, gru_head_newton, gru_head_sequential
from oracle.slstm import SLSTMParams, slstm_newton, slstm_sequential


def _segments(cu_seqlens: Tensor) -> list[tuple[int, int]]:
    cs = cu_seqlens.tolist()
    return [(cs[i], cs[i + 1]) for i in range(len(cs) - 1)]


def slstm_newton_ragged(p: SLSTMParams, x: Tensor, cu_seqlens: Tensor, *, max_iters: int,
                        picard_iters: int, h0: Tensor | None = None) -> Tensor:
    parts = []
    for s, (a, b) in enumerate(_segments(cu_seqlens)):
        hs = None if h0 is None else h0[s:s + 1]
        parts.append(slstm_newton(p, x[:, a:b], max_iters=max_iters, picard_iters=picard_iters,
                                  h0=hs))
    return torch.cat(parts, dim=1)


def slstm_sequential_ragged(p: SLSTMParams, x: Tensor, cu_seqlens: Tensor,
                            h0: Tensor | None = None) -> Tensor:
    parts = [slstm_sequential(p, x[:, a:b], None if h0 is None else h0[s:s + 1])
             for s, (a, b) in enumerate(_segments(cu_seqlens))]
    return torch.cat(parts, dim=1)


def gru_head_newton_ragged(p: GRUHeadParams, x: Tensor, cu_seqlens: Tensor, *,
                           max_iters: int, h0: Tensor | None = None) -> Tensor:
    parts = [gru_head_newton(p, x[:, a:b], max_iters=max_iters,
                             h0=None if h0 is None else h0[s:s + 1])
             for s, (a, b) in enumerate(_segments(cu_seqlens))]
    return torch.cat(parts, dim=1)


def gru_head_sequential_ragged(p: GRUHeadParams, x: Tensor, cu_seqlens: Tensor,
                               h0: Tensor | None = None) -> Tensor:
    parts = [gru_head_sequential(p, x[:, a:b], None if h0 is None else h0[s:s + 1])
             for s, (a, b) in enumerate(_segments(cu_seqlens))]
    return torch.cat(parts, dim=1)
