"""Packed ragged batches (``cu_seqlens``) and paged ``h0`` (``block_table``).

The reference packs S sequences into one stream ``(1, N, ...)`` with
FlashAttention-style offsets ``cu_seqlens`` ``(S+1,)`` and drops the carry at
each sequence head (J = 0 there, ``h0[s]`` as the previous state;
``layout.py:93-138``, ``solvers/scan.py:206-216``).

The diag-sLSTM kernels do exactly that on the packed stream itself (head
flags inside the scans, ``block_table`` read by the kernels; see
``ops.slstm_init_fused`` / ``ops.newton_slstm_fused``).  This module holds the
host rules shared by every path (offset checks, the ragged prepend, the
``block_table`` gather) and the padded route that the other cells take, and
the diag sLSTM with ``PARARNN_AMD_PACKED=0``: sequences never interact, so
they can run as a padded rectangular batch ``(S, T_max, ...)`` through the
same fused kernels.  Every sequence then starts from its own ``h0`` exactly
as at a head, positions past a sequence's end are computed and discarded
(they come after it in time, so they cannot reach it), and the result is
gathered back into the packed order.  Padding and gathering are
differentiable index operations, so the eq. 2.6 backward runs unchanged (the
upstream gradient at discarded positions is zero, so nothing flows from them).

When lengths are uneven, one rectangle would cost ``S * T_max`` steps for
``N`` tokens (a single long sequence among many short ones: orders of
magnitude).  ``RaggedPlan`` therefore sorts the sequences by length and splits
them into groups in which no sequence is padded to more than twice its length
(or by more than 256 steps); each group is its own padded batch (one fused
solve), so the padded work stays below ``2 N + 256 S`` plus one launch set per
group (at most ``log2(T_max / 256) + 2`` groups).
"""

from __future__ import annotations

import os
import weakref

import torch
from torch import Tensor


# The last offsets that passed the checks: weak references to the tensor given
# and to the int64 one returned, each with its version counter (bumped by every
# in-place write), so the solve and the ops it calls check one stream once,
# with one device-to-host copy.
_checked: tuple[tuple[tuple[weakref.ref, int], ...], int] | None = None


def _known(t: Tensor, time: int) -> bool:
    c = _checked
    return c is not None and c[1] == time and any(r() is t and v == t._version for r, v in c[0])


def packed_in_kernel() -> bool:
    """Packed streams run in the kernels (heads cut the carry; diag sLSTM and
    head GRU); ``PARARNN_AMD_PACKED=0`` pads them into length groups instead."""
    return os.environ.get("PARARNN_AMD_PACKED", "1") != "0"


def validate_cu_seqlens(cu_seqlens: Tensor, time: int,
                        device: torch.device | None = None) -> Tensor:
    """``(S+1,)`` exclusive prefix with ``[0] = 0``, last = ``time``, strictly increasing
    (layout.py:93-104); returned as int64 on ``device`` (default: where it is)."""
    global _checked
    if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
        raise ValueError(f"cu_seqlens must be (S+1,), got {tuple(cu_seqlens.shape)}")
    cs = cu_seqlens.to(dtype=torch.long, device=device or cu_seqlens.device)
    if _known(cu_seqlens, time) or _known(cs, time):
        return cs
    host = cs.cpu()
    if int(host[0]) != 0:
        raise ValueError(f"cu_seqlens[0] must be 0, got {int(host[0])}")
    if int(host[-1]) != int(time):
        raise ValueError(f"cu_seqlens[-1] must equal time={time}, got {int(host[-1])}")
    if bool((host[1:] <= host[:-1]).any()):
        raise ValueError("cu_seqlens must be strictly increasing")
    _checked = (tuple((weakref.ref(t), t._version) for t in {id(cu_seqlens): cu_seqlens,
                                                             id(cs): cs}.values()), int(time))
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
    """Index maps between a packed stream ``(1, N, ...)`` and ``(S, T_max, ...)``.

    ``seqs`` (optional, sequence ids) restricts the rectangle to those
    sequences, in that order; ``positions`` holds the packed position of each
    element ``unpad`` returns."""

    def __init__(self, cs: Tensor, device: torch.device, seqs: Tensor | None = None) -> None:
        cs = cs.to(device)
        starts, lengths = cs[:-1], cs[1:] - cs[:-1]
        if seqs is not None:
            seqs = seqs.to(device)
            starts, lengths = starts[seqs], lengths[seqs]
        self.n_seq = int(lengths.numel())
        self.t_max = int(lengths.max())
        self.n = int(cs[-1])
        steps = torch.arange(self.t_max, device=device)
        self.mask = steps[None, :] < lengths[:, None]  # (S, T_max)
        self.index = (starts[:, None] + steps[None, :]).clamp(max=self.n - 1)
        self.positions = self.index[self.mask]
        # Rows of the flattened (S * T_max) rectangle that hold real steps, in
        # the order of ``positions`` (a first-dimension gather, the fast path
        # of torch's indexing, unlike a boolean mask over two dimensions).
        self.rows = self.mask.flatten().nonzero().squeeze(1)
        # One sequence: the rectangle is a slice of the packed stream (a view).
        self.span = (int(starts[0]), int(starts[0]) + self.t_max) if self.n_seq == 1 else None

    def pad(self, packed: Tensor) -> Tensor:
        """``(1, N, ...)`` -> ``(S, T_max, ...)`` with zeros past each sequence's end."""
        if self.span is not None:
            return packed[:, self.span[0]:self.span[1]]
        g = packed[0][self.index]
        m = self.mask.reshape(*self.mask.shape, *([1] * (g.dim() - 2)))
        return torch.where(m, g, torch.zeros((), dtype=g.dtype, device=g.device))

    def unpad(self, padded: Tensor) -> Tensor:
        """``(S, T_max, ...)`` -> ``(1, n, ...)``, the rectangle's own steps in
        packed order (``positions``)."""
        if self.span is not None:
            return padded
        return padded.flatten(0, 1)[self.rows].unsqueeze(0)


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


def length_groups(lengths: list[int], ratio: float = 2.0, slack: int = 256) -> list[list[int]]:
    """Sequence ids grouped by length: longest first, a group closing when the
    next length is below ``1 / ratio`` of the group's longest and more than
    ``slack`` steps short of it (so a sequence of length l is padded to at
    most ``max(ratio * l, l + slack)`` steps; short sequences share a group
    instead of each costing a launch set)."""
    order = sorted(range(len(lengths)), key=lambda i: (-lengths[i], i))
    groups: list[list[int]] = []
    top = None
    for i in order:
        if top is None or (lengths[i] * ratio < top and top - lengths[i] > slack):
            groups.append([])
            top = lengths[i]
        groups[-1].append(i)
    return groups


class RaggedPlan:
    """A packed batch as one or more padded rectangles (length groups).

    ``run(packed, h0, solve)`` calls ``solve(padded, h0_rows)`` once per group
    (``padded`` of shape ``(S_g, T_g, ...)``, ``h0_rows`` the group's rows of
    ``h0`` or None) and returns the solved states in packed order
    ``(1, N, ...)``; every step is an index operation, so autograd flows
    through it.  ``PARARNN_AMD_RAGGED_GROUPS=0`` keeps a single rectangle."""

    def __init__(self, cs: Tensor, device: torch.device, ratio: float = 2.0) -> None:
        lengths = (cs[1:] - cs[:-1]).tolist()
        self.n_seq = len(lengths)
        if os.environ.get("PARARNN_AMD_RAGGED_GROUPS", "1") == "0":
            groups = [list(range(self.n_seq))]
        else:
            groups = length_groups(lengths, ratio)
        if len(groups) == 1:
            self.seqs = [None]
            self.pads = [Padding(cs, device)]
            self.scatter = False  # one rectangle
        else:
            self.seqs = [torch.tensor(g, dtype=torch.long, device=device) for g in groups]
            self.pads = [Padding(cs, device, s) for s in self.seqs]
            self.scatter = True  # groups gathered into the packed output
            # source[i]: row of the concatenated flattened rectangles holding
            # packed step i (every step belongs to exactly one group).
            n = self.pads[0].n
            source = torch.empty(n, dtype=torch.long, device=device)
            off = 0
            for pad in self.pads:
                source[pad.positions] = pad.rows + off
                off += pad.n_seq * pad.t_max
            self.source = source
        self.padded_steps = sum(p.n_seq * p.t_max for p in self.pads)

    @property
    def n_groups(self) -> int:
        return len(self.pads)

    def run(self, packed: Tensor, h0: Tensor | None, solve) -> Tensor:
        if not self.scatter:
            return self.pads[0].unpad(solve(self.pads[0].pad(packed), h0))
        buf, off = None, 0
        for pad, seqs in zip(self.pads, self.seqs):
            part = solve(pad.pad(packed), None if h0 is None else h0[seqs]).flatten(0, 1)
            if buf is None:
                total = sum(p.n_seq * p.t_max for p in self.pads)
                buf = part.new_empty((total,) + tuple(part.shape[1:]))
            # contiguous slice copies (plain device copies, unlike torch.cat's
            # batched kernel); autograd flows through them
            buf[off:off + part.shape[0]] = part
            off += part.shape[0]
        return buf[self.source].unsqueeze(0)
