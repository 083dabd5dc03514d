"""Sequential unroll — the numerics oracle that ``verify_agreement`` compares
against (reference ``solvers/sequential.py:22-86``).  Plain torch ops on the
tensors' device: one shared ``W_x`` GEMM, then ``cell.step`` over T; a single
step without autograd on the GPU goes through ``decode_step``.
"""

from __future__ import annotations

import inspect

import torch
from torch import Tensor, nn


def _zero_state(cell: nn.Module, batch: int, ref: Tensor) -> Tensor:
    slots = getattr(cell, "state_slots", 1)
    if slots == 1:
        return ref.new_zeros(batch, cell.d_h)
    return ref.new_zeros(batch, slots, cell.d_h)


def sequential_apply(cell: nn.Module, x: Tensor, h0: Tensor | None = None, *, step=None,
                     cu_seqlens: Tensor | None = None) -> Tensor:
    """Unroll ``cell.step`` along time; output at t is the state after step t."""
    if cu_seqlens is not None:
        return _sequential_ragged(cell, x, h0, step=step, cu_seqlens=cu_seqlens)
    batch, time, _ = x.shape
    if time < 1:
        raise ValueError(f"sequential_apply needs time >= 1, got {time}")
    h = h0 if h0 is not None else _zero_state(cell, batch, x)
    fn = step or cell.step
    wx_all = None
    if step is None and "wx" in inspect.signature(cell.step).parameters:
        lin = getattr(cell, "W_x", None)
        if lin is not None:
            wx_all = lin(x)
    if step is None and time == 1 and not torch.is_grad_enabled():
        from pararnn_amd.decode import can_decode_step, decode_step

        if can_decode_step(cell, x):
            # T = 1 without autograd: the decode kernel (sequential.py:77-81)
            wx_t = None if wx_all is None else wx_all[:, 0]
            return decode_step(cell, h, x[:, 0], wx=wx_t).unsqueeze(1)
    outs = []
    for t in range(time):
        h = fn(h, x[:, t]) if wx_all is None else fn(h, x[:, t], wx=wx_all[:, t])
        outs.append(h)
    return torch.stack(outs, dim=1)


def _sequential_ragged(cell: nn.Module, x: Tensor, h0: Tensor | None, *, step,
                       cu_seqlens: Tensor) -> Tensor:
    """Packed ``(1, N, d_in)``: each sequence unrolled from ``h0[s]`` (or zeros)."""
    from pararnn_amd.ragged import validate_cu_seqlens

    if x.shape[0] != 1:
        raise ValueError(f"cu_seqlens packs x with batch=1, got batch={x.shape[0]}")
    cs = validate_cu_seqlens(cu_seqlens, x.shape[1]).tolist()
    if h0 is not None and h0.shape[0] != len(cs) - 1:
        raise ValueError(f"h0 batch {h0.shape[0]} != n_seq {len(cs) - 1}")
    parts = []
    for s in range(len(cs) - 1):
        hs = None if h0 is None else h0[s:s + 1]
        parts.append(sequential_apply(cell, x[:, cs[s]:cs[s + 1]], hs, step=step))
    return torch.cat(parts, dim=1)
