"""T=1 decode for the serving loop (reference ``kernels/decode.py:119-597``).

``decode_step(cell, state, x, wx=, out=, block_table=)`` advances one step.
On a ROCm GPU without autograd it runs one HIP kernel for the recurrent part
of ``cell.step`` (``ParaSLSTM(mix='diag')``, ``ParaGRU(mix='diag'|'head')``);
``W_x(x)`` stays a library GEMM (``decode_wx``).  Elsewhere (CPU tensors,
autograd, other cells) it runs the cell's own ``step`` with torch ops, as the
reference does.  ``block_table`` (``(B,)`` slot ids) reads and writes a
pool-shaped state in place; ``out=`` reuses a buffer.  The recurrent
parameters are clamped inside the kernel, so a captured graph allocates
nothing.
"""

from __future__ import annotations

import inspect

import torch
from torch import Tensor, nn

from pararnn_amd import _lib
from pararnn_amd.cells import ParaGRU, ParaSLSTM
from pararnn_amd.head_blocks import HeadBlocks
from pararnn_amd.ops import _ptr, _stream, _validate


def can_decode_step(cell: nn.Module, ref: Tensor) -> bool:
    """Whether ``decode_step`` runs the HIP kernel for ``cell`` on ``ref``'s device/dtype."""
    if ref.device.type != "cuda" or ref.dtype not in (torch.float32, torch.bfloat16,
                                                      torch.float16):
        return False
    if isinstance(cell, ParaSLSTM):
        return cell.mix == "diag"
    if isinstance(cell, ParaGRU):
        return cell.mix == "diag" or (cell.mix == "head" and _head_blocks_in_place(cell))
    return False


def _head_blocks_in_place(cell: ParaGRU) -> bool:
    """Heads that tile 64-channel blocks exactly (d_head = 64, or a divisor of
    64 with whole blocks of heads): the kernel then reads and writes the state
    in place, merged heads being block-diagonal 64 x 64 matrices."""
    d_head = int(cell.d_head)
    return d_head <= 64 and 64 % d_head == 0 and int(cell.n_heads) % (64 // d_head) == 0


def _squeeze_time(t: Tensor, name: str) -> Tensor:
    if t.dim() == 3:
        if t.shape[1] != 1:
            raise ValueError(f"decode_step {name} time dim must be 1, got {tuple(t.shape)}")
        return t[:, 0]
    if t.dim() != 2:
        raise ValueError(f"decode_step {name} needs (B, features), got {tuple(t.shape)}")
    return t


def decode_wx(cell: nn.Module, x: Tensor, *, out: Tensor | None = None) -> Tensor:
    """``W_x(x)`` for one step, optionally into ``out`` (decode.py:77-110)."""
    lin = getattr(cell, "W_x", None)
    if lin is None:
        raise TypeError(f"decode_wx needs cell.W_x; got {type(cell).__name__}")
    x2 = _squeeze_time(x, "x")
    if out is None:
        return lin(x2)
    torch.mm(x2, lin.weight.t(), out=out)
    if lin.bias is not None:
        out.add_(lin.bias)
    return out


def _accepts_wx(cell: nn.Module) -> bool:
    step = getattr(cell, "step", None)
    try:
        return step is not None and "wx" in inspect.signature(step).parameters
    except (TypeError, ValueError):
        return False


def _is_capturing() -> bool:
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def _resolve_out(state: Tensor, out: Tensor | None, block_table: Tensor | None):
    if block_table is None:
        if out is None:
            out = torch.empty_like(state)
        elif out.shape != state.shape:
            raise ValueError(
                f"decode_step out shape {tuple(out.shape)} != state {tuple(state.shape)}")
        elif out.dtype != state.dtype or out.device != state.device:
            raise ValueError("decode_step out must match state dtype and device")
        return out, None, int(state.shape[0])
    bt = block_table.to(device=state.device, dtype=torch.int32).contiguous()
    if bt.dim() != 1:
        raise ValueError(f"block_table must be 1-D (B,), got {tuple(bt.shape)}")
    if out is None:
        out = state
    elif out.shape != state.shape:
        raise ValueError("block_table decode writes pool-shaped out "
                         f"(same as state {tuple(state.shape)}), got {tuple(out.shape)}")
    elif out.dtype != state.dtype or out.device != state.device:
        raise ValueError("decode_step out must match state dtype and device")
    return out, bt, int(bt.numel())


def decode_step(cell: nn.Module, state: Tensor, x: Tensor | None = None, *,
                wx: Tensor | None = None, out: Tensor | None = None,
                block_table: Tensor | None = None) -> Tensor:
    """One recurrent step; returns the next state (``out`` when given)."""
    ref = wx if wx is not None else x
    if ref is None:
        raise ValueError("decode_step needs x or wx (precomputed W_x(x))")
    if not (can_decode_step(cell, ref) and not torch.is_grad_enabled()):
        if block_table is not None:
            raise RuntimeError("block_table requires the GPU decode_step kernel")
        y = cell.step(state, x, wx=wx) if _accepts_wx(cell) else cell.step(state, x)
        if out is None:
            return y
        out.copy_(y)
        return out
    if wx is None:
        wx = decode_wx(cell, x)
    wx = _squeeze_time(wx, "wx")
    if _is_capturing():
        if not state.is_contiguous() or not wx.is_contiguous():
            raise RuntimeError("decode_step under graph capture needs contiguous state and wx")
        if out is None and block_table is None:
            raise RuntimeError("decode_step under graph capture needs out= (or block_table)")
    elif not state.is_contiguous():
        state = state.contiguous()
    if not wx.is_contiguous():
        wx = wx.contiguous()
    out, bt, batch = _resolve_out(state, out, block_table)
    if wx.shape[0] != batch:
        raise ValueError(f"decode_step wx batch {wx.shape[0]} != {batch}")
    cap = cell.max_recurrent_norm
    has_cap = int(cap is not None)
    capf = float(cap) if cap is not None else 0.0
    d = int(cell.d_h)
    lib = _lib.load()
    if isinstance(cell, ParaSLSTM):
        if wx.shape[-1] != 4 * d:
            raise ValueError(f"ParaSLSTM wx last dim {wx.shape[-1]} != 4 * d_h={4 * d}")
        code = _validate("decode_slstm", state, wx, cell.R, out)
        with torch.cuda.device(state.device):
            rc = lib.prnn_slstm_decode(
                _ptr(state), _ptr(wx), _ptr(cell.R.contiguous()), _ptr(out), _ptr(bt), batch, d,
                float(cell.eps), capf, has_cap, code, _stream(state.device))
        _lib.check(rc, "decode_slstm")
        return out
    if cell.mix == "diag":
        a = (cell.a_z, cell.a_r, cell.a_n)
        heads = 0
    else:
        hb = HeadBlocks(int(cell.n_heads), int(cell.d_head), state.device)
        a = tuple(hb.matrices(t) for t in (cell.A_z, cell.A_r, cell.A_n))
        heads = hb.n_blocks
    if wx.shape[-1] != 3 * d:
        raise ValueError(f"ParaGRU wx last dim {wx.shape[-1]} != 3 * d_h={3 * d}")
    code = _validate("decode_gru", state, wx, *a, out)
    a = tuple(t.contiguous() for t in a)
    with torch.cuda.device(state.device):
        rc = lib.prnn_gru_decode(
            _ptr(state), _ptr(wx), _ptr(a[0]), _ptr(a[1]), _ptr(a[2]), _ptr(out), _ptr(bt),
            batch, d, heads, capf, has_cap, code, _stream(state.device))
    _lib.check(rc, "decode_gru")
    return out
