"""Heads narrower than 64 channels on the 64-channel head-GRU kernels.

The head-GRU kernels work on blocks of 64 channels whose recurrent matrices
are 64 x 64 (the matrix-core tile).  A cell with ``d_head < 64`` has
block-diagonal recurrent weights with smaller blocks; several of its heads fit
in one 64-channel block whose 64 x 64 matrix is block-diagonal with the heads'
matrices on the diagonal and zeros elsewhere.  The GRU step and its Jacobian
then act on each head exactly as the narrow head would: products with the zero
off-diagonal blocks contribute exact zeros.

Layout.  ``per = 64 // d_head`` heads share a block; head ``h`` sits in block
``h // per`` at channel offset ``(h % per) * d_head``.  When ``64 % d_head ==
0`` and the heads fill whole blocks, that is the identity map on channels, so
``wx``, ``h0`` and the outputs are used as they are (no copies).  Otherwise
(``d_head`` not dividing 64, or a partly filled last block) the channels are
scattered into a zero-padded block layout and gathered back; padded channels
have zero inputs, zero weights and zero initial state, so they stay at zero
(z = r = 1/2, n = 0 gives h' = h / 2) and never touch a real channel.

The reference handles ``d_head <= 64`` with a masked ``BLOCK_D`` tile
(kernels/newton_gru_head.py:121-136).  Heads of 64 < d_head <= 128 take the
wide tier instead (``ops._gru_head_wide``), not these blocks.

Caveat of sharing a block: the matrix-core products multiply the zero
off-diagonal entries too, so a non-finite value in one narrow head's state
or gradient (inf * 0 = NaN) reaches the other heads of its block, where the
reference's masked tile keeps heads apart.  Finite inputs are unaffected.
"""

from __future__ import annotations

import torch
from torch import Tensor

BLOCK = 64


class HeadBlocks:
    """Placement of ``n_heads`` heads of ``d_head`` channels in 64-channel blocks."""

    def __init__(self, n_heads: int, d_head: int, device: torch.device) -> None:
        if not 1 <= d_head <= BLOCK:
            raise TypeError(f"head GRU kernels take 1 <= d_head <= {BLOCK}, got {d_head}")
        self.n_heads = n_heads
        self.d_head = d_head
        self.per = BLOCK // d_head
        self.n_blocks = -(-n_heads // self.per)
        self.d_h = n_heads * d_head
        self.d_pad = self.n_blocks * BLOCK
        self.identity = BLOCK % d_head == 0 and n_heads % self.per == 0
        if d_head != BLOCK:
            # flat position in (n_blocks, 64, 64) of every (head, row, col)
            h = torch.arange(n_heads, device=device).view(-1, 1, 1)
            i = torch.arange(d_head, device=device).view(1, -1, 1)
            j = torch.arange(d_head, device=device).view(1, 1, -1)
            off = (h % self.per) * d_head
            self.flat = ((h // self.per) * BLOCK * BLOCK + (off + i) * BLOCK + off + j).reshape(-1)
        if not self.identity:
            head = torch.arange(n_heads, device=device).repeat_interleave(d_head)
            within = torch.arange(d_head, device=device).repeat(n_heads)
            # padded channel of every real channel
            self.chan = (head // self.per) * BLOCK + (head % self.per) * d_head + within

    # -- weights ---------------------------------------------------------------

    def matrices(self, a: Tensor) -> Tensor:
        """``(n_heads, d_head, d_head)`` -> ``(n_blocks, 64, 64)`` block-diagonal."""
        if self.d_head == BLOCK:
            return a.contiguous()
        out = a.new_zeros(self.n_blocks * BLOCK * BLOCK)
        out.index_copy_(0, self.flat, a.reshape(-1))
        return out.view(self.n_blocks, BLOCK, BLOCK)

    def head_grads(self, g: Tensor) -> Tensor:
        """Gradients ``(G, n_blocks, 64, 64)`` -> ``(G, n_heads, d_head, d_head)``
        (the diagonal blocks; the zero off-diagonal entries are structural)."""
        if self.d_head == BLOCK:
            return g
        gates = g.shape[0]
        return g.reshape(gates, -1).index_select(1, self.flat).view(
            gates, self.n_heads, self.d_head, self.d_head)

    # -- activations -----------------------------------------------------------

    def to_blocks(self, t: Tensor | None, gates: int = 1) -> Tensor | None:
        """``(..., gates * d_h)`` -> ``(..., gates * d_pad)`` (zero padding)."""
        if t is None or self.identity:
            return t
        lead = t.shape[:-1]
        src = t.reshape(*lead, gates, self.d_h)
        out = t.new_zeros(*lead, gates, self.d_pad)
        out.index_copy_(-1, self.chan, src)
        return out.reshape(*lead, gates * self.d_pad)

    def from_blocks(self, t: Tensor | None, gates: int = 1) -> Tensor | None:
        """``(..., gates * d_pad)`` -> ``(..., gates * d_h)``."""
        if t is None or self.identity:
            return t
        lead = t.shape[:-1]
        return t.reshape(*lead, gates, self.d_pad).index_select(-1, self.chan).reshape(
            *lead, gates * self.d_h)
