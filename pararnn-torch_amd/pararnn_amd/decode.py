"""T=1 decode for the serving loop (public surface of reference ``kernels/decode.py:119-270``).

``decode_step(cell, state, x, wx=, out=, block_table=)`` advances every row
of a batch by one step and returns the next state.

How a call is served:

* **kernel** -- a ROCm tensor of a supported dtype, no autograd, and a cell
  with a decode kernel (``ParaSLSTM(mix='diag')``, ``ParaGRU(mix='diag')``,
  ``ParaGRU(mix='head')`` whose heads tile 64-channel blocks): one HIP launch
  computes the recurrent part of the step from the pre-projected gates
  ``wx = W_x(x)`` (a library GEMM, :func:`decode_wx`, when only ``x`` is
  given).  The recurrent parameters are clamped inside the kernel, so a
  captured graph holds no clamp ops and allocates nothing.
* **torch** -- anything else runs the cell's own ``step`` (CPU tensors, an
  autograd step, cells without a kernel).  A block table needs the kernel.

``block_table`` ``(B,)`` names, for batch row b, the pool row the kernel reads
and overwrites in place (``state`` is the pool; ``out`` defaults to it);
without it the next state goes to ``out`` or a new tensor.  Under HIP graph
capture every operand must already be laid out contiguously and the
destination must exist (``out=`` or a block table): nothing is copied or
allocated inside a captured step.
"""

from __future__ import annotations

import weakref
from typing import NamedTuple

import torch
from torch import Tensor, nn

from pararnn_amd import _lib
from pararnn_amd.cells import ParaGRU, ParaSLSTM
from pararnn_amd.head_blocks import HeadBlocks
from pararnn_amd.ops import _ptr, _stream, _validate

_KERNEL_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _kernel_kind(cell: nn.Module) -> str | None:
    """'slstm' / 'gru' when a decode kernel exists for the cell's structure."""
    if isinstance(cell, ParaSLSTM) and cell.mix == "diag":
        return "slstm"
    if isinstance(cell, ParaGRU):
        if cell.mix == "diag":
            return "gru"
        if cell.mix == "head":
            d_head, n_heads = int(cell.d_head), int(cell.n_heads)
            # merged heads must fill whole 64-channel blocks so that the state
            # rows are already in the kernel's layout (read and written in place)
            if d_head <= 64 and 64 % d_head == 0 and n_heads % (64 // d_head) == 0:
                return "gru"
    return None


def can_decode_step(cell: nn.Module, ref: Tensor) -> bool:
    """Whether ``decode_step`` runs the HIP kernel for ``cell`` on ``ref``'s device/dtype."""
    return (ref.device.type == "cuda" and ref.dtype in _KERNEL_DTYPES
            and _kernel_kind(cell) is not None)


def _one_step(t: Tensor, what: str) -> Tensor:
    """``(B, 1, F)`` or ``(B, F)`` -> ``(B, F)``."""
    if t.dim() == 2:
        return t
    if t.dim() == 3 and t.shape[1] == 1:
        return t[:, 0]
    raise ValueError(f"decode_step {what} must be (B, F) or (B, 1, F), got {tuple(t.shape)}")


def decode_wx(cell: nn.Module, x: Tensor, *, out: Tensor | None = None) -> Tensor:
    """``W_x(x)`` for one step, written into ``out`` when given (decode.py:77-110)."""
    proj = getattr(cell, "W_x", None)
    if proj is None:
        raise TypeError(f"decode_wx needs cell.W_x; got {type(cell).__name__}")
    rows = _one_step(x, "x")
    if out is None:
        return proj(rows)
    if proj.bias is None:
        return torch.mm(rows, proj.weight.t(), out=out)
    return torch.addmm(proj.bias, rows, proj.weight.t(), out=out)


# -- operands of one kernel launch ------------------------------------------------


class _Target(NamedTuple):
    """Where the kernel reads the previous state and writes the next one."""

    out: Tensor
    table: Tensor | None  # int32 pool rows, one per batch row
    rows: int  # batch rows advanced by the step


def _laid_out(t: Tensor, what: str, capturing: bool) -> Tensor:
    if t.is_contiguous():
        return t
    if capturing:
        raise RuntimeError(f"decode_step under graph capture needs a contiguous {what}")
    return t.contiguous()


def _target(state: Tensor, out: Tensor | None, block_table: Tensor | None,
            capturing: bool) -> _Target:
    if out is not None:
        if out.shape != state.shape:
            raise ValueError(f"decode_step out {tuple(out.shape)} must have the shape of state "
                             f"{tuple(state.shape)}")
        if out.dtype != state.dtype or out.device != state.device:
            raise ValueError("decode_step out must match state dtype and device")
    if block_table is None:
        if out is None:
            if capturing:
                raise RuntimeError("decode_step under graph capture needs out= (or a "
                                   "block_table)")
            out = torch.empty_like(state)
        return _Target(out, None, int(state.shape[0]))
    if block_table.dim() != 1:
        raise ValueError(f"block_table must be 1-D (B,), got {tuple(block_table.shape)}")
    table = block_table
    if table.dtype != torch.int32 or table.device != state.device:
        if capturing:
            raise RuntimeError("decode_step under graph capture needs an int32 block_table on "
                               "the state's device")
        table = table.to(device=state.device, dtype=torch.int32)
    return _Target(state if out is None else out, _laid_out(table, "block_table", capturing),
                   int(table.numel()))


# Block-diagonal 64 x 64 recurrent matrices of head GRUs with d_head < 64, kept
# per cell and rebuilt only when a parameter changes (its version counter or
# storage), so a decode step of such a cell launches the kernel alone.
_head_mats: weakref.WeakKeyDictionary = weakref.WeakKeyDictionary()


def _gru_recurrent(cell: ParaGRU) -> tuple[tuple[Tensor, Tensor, Tensor], int]:
    """The three recurrent operands and the number of 64-channel blocks (0 = diag)."""
    if cell.mix == "diag":
        return (cell.a_z, cell.a_r, cell.a_n), 0
    params = (cell.A_z, cell.A_r, cell.A_n)
    if int(cell.d_head) == 64:
        return tuple(p.contiguous() for p in params), int(cell.n_heads)
    key = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in params)
    hit = _head_mats.get(cell)
    if hit is None or hit[0] != key:
        blocks = HeadBlocks(int(cell.n_heads), int(cell.d_head), params[0].device)
        with torch.no_grad():
            mats = tuple(blocks.matrices(p.detach()) for p in params)
        hit = (key, mats, blocks.n_blocks)
        _head_mats[cell] = hit
    return hit[1], hit[2]


def _launch(cell: nn.Module, kind: str, state: Tensor, gates: Tensor, tgt: _Target) -> None:
    lib = _lib.load()
    d = int(cell.d_h)
    cap = cell.max_recurrent_norm
    clamp = (0.0, 0) if cap is None else (float(cap), 1)
    table = None if tgt.table is None else _ptr(tgt.table)
    if kind == "slstm":
        if gates.shape[-1] != 4 * d:
            raise ValueError(f"ParaSLSTM wx last dim {gates.shape[-1]} != 4 * d_h={4 * d}")
        r = cell.R if cell.R.is_contiguous() else cell.R.contiguous()
        code = _validate("decode_slstm", state, gates, r, tgt.out)
        with torch.cuda.device(state.device):
            rc = lib.prnn_slstm_decode(_ptr(state), _ptr(gates), _ptr(r), _ptr(tgt.out), table,
                                       tgt.rows, d, float(cell.eps), *clamp, code,
                                       _stream(state.device))
        _lib.check(rc, "decode_slstm")
        return
    if gates.shape[-1] != 3 * d:
        raise ValueError(f"ParaGRU wx last dim {gates.shape[-1]} != 3 * d_h={3 * d}")
    (a_z, a_r, a_n), blocks = _gru_recurrent(cell)
    code = _validate("decode_gru", state, gates, a_z, a_r, a_n, tgt.out)
    with torch.cuda.device(state.device):
        rc = lib.prnn_gru_decode(_ptr(state), _ptr(gates), _ptr(a_z), _ptr(a_r), _ptr(a_n),
                                 _ptr(tgt.out), table, tgt.rows, d, blocks, *clamp, code,
                                 _stream(state.device))
    _lib.check(rc, "decode_gru")


def decode_step(cell: nn.Module, state: Tensor, x: Tensor | None = None, *,
                wx: Tensor | None = None, out: Tensor | None = None,
                block_table: Tensor | None = None) -> Tensor:
    """Advance ``state`` by one step; returns the next state (``out`` when given).

    ``x`` ``(B, d_in)`` (or ``(B, 1, d_in)``) or the precomputed ``wx`` (same
    with ``G * d_h`` features) supplies the step's input.
    """
    if x is None and wx is None:
        raise ValueError("decode_step needs x or wx (precomputed W_x(x))")
    probe = x if wx is None else wx
    kind = _kernel_kind(cell)
    if (kind is None or torch.is_grad_enabled() or probe.device.type != "cuda"
            or probe.dtype not in _KERNEL_DTYPES):
        if block_table is not None:
            raise RuntimeError("block_table requires the GPU decode_step kernel")
        nxt = cell.step(state, x) if wx is None else cell.step(state, x, wx=wx)
        return nxt if out is None else out.copy_(nxt)
    capturing = torch.cuda.is_current_stream_capturing()
    gates = _one_step(decode_wx(cell, x) if wx is None else wx, "wx")
    gates = _laid_out(gates, "wx", capturing)
    state = _laid_out(state, "state", capturing)
    tgt = _target(state, out, block_table, capturing)
    if gates.shape[0] != tgt.rows:
        raise ValueError(f"decode_step wx has {gates.shape[0]} rows, the step advances "
                         f"{tgt.rows}")
    _launch(cell, kind, state, gates, tgt)
    return tgt.out
