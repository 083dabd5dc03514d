"""``torch.library`` custom ops over the HIP kernels (the drop-in boundary).

``pararnn::newton_slstm_fused`` and ``pararnn::newton_gru_head_fused`` keep the
names, schemas, return layouts and error types of the reference's ops
(``kernels/custom_ops.py:311-386, 486-540``); ``pararnn::slstm_init_fused``
is the frozen-gate / Picard guess that the reference computes in Python
before calling its op (``kernels/fused_newton.py:358-372``).  Each op
validates on the host, allocates its outputs and a workspace through torch's
caching allocator, and enqueues the kernels on the current stream of the
tensors' device through the C ABI.  All are functional (``mutates_args=()``)
and have fake kernels for ``torch.compile``.
"""

from __future__ import annotations

import collections
import ctypes
import os
import threading

import torch
from torch import Tensor

from pararnn_amd import _lib
from pararnn_amd.head_blocks import HeadBlocks

_DTYPES = {torch.float32: _lib.PRNN_F32, torch.bfloat16: _lib.PRNN_BF16,
           torch.float16: _lib.PRNN_F16}


def _validate(name: str, *tensors: Tensor | None) -> int:
    """Device/dtype rules of the reference's ``validate_cuda_tensors``
    (kernels/precision.py:40-68): one GPU device, one dtype, float32/bfloat16/float16."""
    ts = [t for t in tensors if t is not None]
    ref = ts[0]
    for t in ts:
        if t.device.type != "cuda":
            raise RuntimeError(f"{name} requires a ROCm GPU tensor, got {t.device}")
        if t.device != ref.device:
            raise RuntimeError(f"{name}: tensors on different devices ({t.device} vs {ref.device})")
        if t.dtype != ref.dtype:
            raise TypeError(f"{name}: dtype mismatch {t.dtype} vs {ref.dtype}")
    if ref.dtype not in _DTYPES:
        raise TypeError(f"{name} supports float32/bfloat16/float16, got {ref.dtype}")
    return _DTYPES[ref.dtype]


def _ptr(t: Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _workspace(nbytes: int, dev: torch.device) -> Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=dev)


# Tagged sLSTM workspaces: one zero-filled buffer per (device, stream), kept
# across calls, with a growing tag base, so a call skips clearing its
# look-back words (prnn_slstm_*_ex).  Only the library writes these buffers;
# calls on one stream run in order.  Graph capture takes a fresh, cleared
# workspace per call (a replay would repeat captured tags).
_TAG_SPAN = 64           # PRNN_TAG_SPAN
_TAG_BASE_MAX = 1 << 30  # PRNN_TAG_BASE_MAX
_TAGGED_MAX = 4          # cached buffers (least recently used dropped first)
_tagged_lock = threading.Lock()
_tagged: collections.OrderedDict[tuple[int, int], list] = collections.OrderedDict()


def _tagged_enabled() -> bool:
    return os.environ.get("PARARNN_AMD_TAGGED_WS", "1") != "0"


def _slstm_workspace(nbytes: int, dev: torch.device) -> tuple[Tensor, int]:
    """``(workspace, tag_base)`` for an sLSTM call on the current stream."""
    if not _tagged_enabled() or torch.cuda.is_current_stream_capturing():
        return _workspace(nbytes, dev), 0
    stream = torch.cuda.current_stream(dev)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), stream.cuda_stream)
    with _tagged_lock:
        ent = _tagged.get(key)
        if ent is None or ent[0].numel() < nbytes or ent[1] + _TAG_SPAN > _TAG_BASE_MAX:
            # Zero-filled on this stream, ahead of the call that uses it.
            ent = [torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=dev), 1]
            _tagged[key] = ent
        _tagged.move_to_end(key)
        while len(_tagged) > _TAGGED_MAX:
            _tagged.popitem(last=False)  # the stream-ordered allocator frees it safely
        base = ent[1]
        ent[1] += _TAG_SPAN
        return ent[0], base


def _check_lookback(ws: Tensor, what: str) -> None:
    """With ``PARARNN_AMD_CHECK_STATUS=1``: wait for the call and raise
    ``RuntimeError`` if one of its look-back or hand-off waits gave up
    (``prnn_slstm_lookback_status``; the affected outputs are NaN)."""
    if os.environ.get("PARARNN_AMD_CHECK_STATUS", "0") == "0":
        return
    if torch.cuda.is_current_stream_capturing():
        return
    st = ctypes.c_int(0)
    lib = _lib.load()
    _lib.check(lib.prnn_slstm_lookback_status(_ptr(ws), ctypes.byref(st), _stream(ws.device)),
               what)
    if st.value:
        raise RuntimeError(f"{what}: a look-back wait gave up (status {st.value}); the output "
                           f"holds NaN where it did")


def release_workspaces() -> None:
    """Drop the cached sLSTM workspaces (they are re-created on demand)."""
    with _tagged_lock:
        _tagged.clear()


# ---------------------------------------------------------------------------
# ParaSLSTM mix='diag'
# ---------------------------------------------------------------------------


def _slstm_shapes(wx: Tensor, r: Tensor) -> tuple[int, int, int]:
    if wx.dim() != 3:
        raise ValueError(f"wx must be (B, T, 4 d_h), got {tuple(wx.shape)}")
    batch, time, four_d = wx.shape
    d_h = r.shape[-1]
    if r.shape != (4, d_h):
        raise ValueError(f"r shape {tuple(r.shape)} != {(4, d_h)}")
    if four_d != 4 * d_h:
        raise ValueError(f"wx last dim {four_d} != 4 * d_h={4 * d_h}")
    return batch, time, d_h


def _slstm_h0(h0: Tensor | None, batch: int, d_h: int) -> Tensor | None:
    if h0 is None:
        return None
    if h0.shape != (batch, 4, d_h):
        raise ValueError(f"h0 shape {tuple(h0.shape)} != {(batch, 4, d_h)}")
    return h0.contiguous()


def _packed_args(cu_seqlens: Tensor | None, block_table: Tensor | None, wx: Tensor,
                 h0: Tensor | None, d_h: int):
    """Device int32 ``cu_seqlens`` / ``block_table`` of a packed stream and the
    checked ``h0`` (``(S, 4, d)`` per sequence, or a pool that ``block_table``
    indexes), or ``(None, None, 0, h0)`` for a rectangular batch."""
    if cu_seqlens is None:
        return None, None, 0, h0
    from pararnn_amd.ragged import validate_cu_seqlens

    if wx.shape[0] != 1:
        raise ValueError(f"cu_seqlens packs wx with batch=1, got batch={wx.shape[0]}")
    cs = validate_cu_seqlens(cu_seqlens, wx.shape[1])
    n_seq = int(cs.numel()) - 1
    bt = None
    if block_table is not None:
        if h0 is None:
            raise ValueError("block_table needs h0 as a pool (C, ...)")
        bt = block_table.to(device=wx.device, dtype=torch.int32).contiguous()
        if bt.dim() != 1 or int(bt.numel()) != n_seq:
            raise ValueError(f"block_table B={int(bt.numel())} != {n_seq}")
        if h0.shape[1:] != (4, d_h):
            raise ValueError(f"pool h0 tail {tuple(h0.shape[1:])} != {(4, d_h)}")
        host = bt.cpu()
        mn, mx = int(host.min()), int(host.max())
        if mn < 0 or mx >= int(h0.shape[0]):
            raise ValueError(f"block_table slots [{mn}, {mx}] outside pool capacity "
                             f"{int(h0.shape[0])}")
    elif h0 is not None and h0.shape != (n_seq, 4, d_h):
        raise ValueError(f"h0 shape {tuple(h0.shape)} != {(n_seq, 4, d_h)}")
    cs32 = cs.to(device=wx.device, dtype=torch.int32).contiguous()
    return cs32, bt, n_seq, None if h0 is None else h0.contiguous()


@torch.library.custom_op("pararnn::slstm_init_fused", mutates_args=())
def slstm_init_fused(
    wx: Tensor, r: Tensor, h0: Tensor | None = None, cu_seqlens: Tensor | None = None,
    block_table: Tensor | None = None, *, picard_iters: int, eps: float
) -> Tensor:
    """Zero-hidden frozen-gate scan plus ``picard_iters`` Picard passes on the GPU.

    Same result layout and rounding points as the reference's
    ``slstm_picard_init`` / ``slstm_zero_hidden_init`` (solvers/slstm_picard.py:143-181):
    states ``(B, T, 4, d_h)`` in ``wx``'s dtype; between passes the trajectory
    is held in that dtype and ``wx + R * h_prev`` is rounded after each op.
    With ``cu_seqlens`` (``wx`` packed as ``(1, N, 4 d_h)``) every sequence
    restarts from its own ``h0`` row (``block_table[s]`` of a pool when given)
    inside the kernels, as the reference's ragged frozen-gate scan does
    (slstm_picard.py:87-103).
    """
    batch, time, d_h = _slstm_shapes(wx, r)
    code = _validate("slstm_init_fused", wx, r, h0)
    if picard_iters < 0:
        raise ValueError(f"n_picard must be >= 0, got {picard_iters!r}")
    wx = wx.contiguous()
    r = r.contiguous()
    cs32, bt, n_seq, h0 = _packed_args(cu_seqlens, block_table, wx, h0, d_h)
    if cs32 is None:
        h0 = _slstm_h0(h0, batch, d_h)
    out = wx.new_empty(batch, time, 4, d_h)
    lib = _lib.load()
    _lib.sync_deterministic(lib)
    with torch.cuda.device(wx.device):
        if cs32 is None:
            nbytes = lib.prnn_slstm_init_workspace_size(batch, time, d_h, picard_iters, code)
            ws, tag = _slstm_workspace(nbytes, wx.device)
            rc = lib.prnn_slstm_init_ex(
                _ptr(wx), _ptr(r), _ptr(h0), _ptr(out), batch, time, d_h, int(picard_iters),
                float(eps), code, _ptr(ws), ws.numel(), tag, _stream(wx.device),
            )
        else:
            nbytes = lib.prnn_slstm_init_packed_workspace_size(time, d_h, picard_iters, code)
            ws, tag = _slstm_workspace(nbytes, wx.device)
            rc = lib.prnn_slstm_init_packed(
                _ptr(wx), _ptr(r), _ptr(h0), _ptr(out), time, d_h, int(picard_iters),
                float(eps), code, _ptr(cs32), n_seq, _ptr(bt), _ptr(ws), ws.numel(), tag,
                _stream(wx.device),
            )
    _lib.check(rc, "slstm_init_fused")
    _check_lookback(ws, "slstm_init_fused")
    return out


@slstm_init_fused.register_fake
def _(wx, r, h0=None, cu_seqlens=None, block_table=None, *, picard_iters, eps):
    batch, time, _ = wx.shape
    return wx.new_empty(batch, time, 4, r.shape[-1])


@torch.library.custom_op("pararnn::newton_slstm_fused", mutates_args=())
def newton_slstm_fused(
    wx: Tensor,
    r: Tensor,
    h0: Tensor | None = None,
    states: Tensor | None = None,
    block_table: Tensor | None = None,
    cu_seqlens: Tensor | None = None,
    *,
    max_iters: int,
    omega: float,
    eps: float,
    log_coords: bool = False,
    scan_tile: str = "assoc",
    time_loop: bool = False,
    window_len: int = 0,
) -> Tensor:
    """``max_iters`` fused Newton iterations for diag ParaSLSTM on the GPU.

    Same schema as the reference op (kernels/custom_ops.py:486-516), plus an
    optional trailing ``cu_seqlens``.  Work is fp32 throughout; intermediate
    trajectories stay fp32 and the result is rounded once to ``wx``'s dtype
    (kernels/newton_slstm.py:2780-2939).  ``states=None`` starts from the
    zero-hidden guess.  With ``cu_seqlens`` (``wx`` packed as ``(1, N, 4 d)``)
    the kernels cut the carry at every sequence head (J = 0 there, the
    sequence's ``h0`` row -- ``block_table[s]`` of a pool when given -- as
    the previous state), the reference's packed semantics
    (solvers/scan.py:206-216, layout.py:115-138), in one stream.
    """
    if log_coords:
        raise TypeError("newton_slstm_fused: log_coords is not provided by pararnn_amd")
    if scan_tile != "assoc":
        raise TypeError(f"newton_slstm_fused: scan_tile={scan_tile!r} is not provided (assoc only)")
    if time_loop or window_len:
        raise TypeError("newton_slstm_fused: fused_time_loop is not provided by pararnn_amd")
    batch, time, d_h = _slstm_shapes(wx, r)
    if block_table is not None and cu_seqlens is None:
        # paged h0 of a rectangular batch: the pool rows the table names
        # (kernels/_fused_common.py:106-139)
        from pararnn_amd.ragged import gather_h0

        h0 = gather_h0(h0, block_table, batch, (4, d_h))
        block_table = None
    code = _validate("newton_slstm_fused", wx, r, h0)
    if max_iters < 0:
        raise ValueError(f"max_iters must be >= 0, got {max_iters!r}")
    cs32, bt, n_seq, h0 = _packed_args(cu_seqlens, block_table, wx, h0, d_h)
    if cs32 is None:
        h0 = _slstm_h0(h0, batch, d_h)
    if states is None:
        states = slstm_init_fused(wx, r, h0, cs32, bt, picard_iters=0, eps=eps)
    else:
        if states.shape != (batch, time, 4, d_h):
            raise ValueError(f"states shape {tuple(states.shape)} != {(batch, time, 4, d_h)}")
        _validate("newton_slstm_fused", wx, states)
    wx = wx.contiguous()
    r = r.contiguous()
    states = states.contiguous()
    out = wx.new_empty(batch, time, 4, d_h)
    lib = _lib.load()
    _lib.sync_deterministic(lib)
    with torch.cuda.device(wx.device):
        if cs32 is None:
            nbytes = lib.prnn_slstm_newton_workspace_size(batch, time, d_h, int(max_iters), code)
            ws, tag = _slstm_workspace(nbytes, wx.device)
            rc = lib.prnn_slstm_newton_ex(
                _ptr(wx), _ptr(r), _ptr(h0), _ptr(states), _ptr(out), batch, time, d_h,
                int(max_iters), float(omega), float(eps), code, _ptr(ws), ws.numel(), tag,
                _stream(wx.device),
            )
        else:
            nbytes = lib.prnn_slstm_newton_packed_workspace_size(time, d_h, int(max_iters), code)
            ws, tag = _slstm_workspace(nbytes, wx.device)
            rc = lib.prnn_slstm_newton_packed(
                _ptr(wx), _ptr(r), _ptr(h0), _ptr(states), _ptr(out), time, d_h,
                int(max_iters), float(omega), float(eps), code, _ptr(cs32), n_seq, _ptr(bt),
                _ptr(ws), ws.numel(), tag, _stream(wx.device),
            )
    _lib.check(rc, "newton_slstm_fused")
    _check_lookback(ws, "newton_slstm_fused")
    return out


def slstm_newton_step(wx: Tensor, r: Tensor, h0: Tensor | None, states: Tensor, *,
                      omega: float, eps: float, cu_seqlens: Tensor | None = None,
                      block_table: Tensor | None = None) -> Tensor:
    """One Newton iteration from ``states`` (``wx``'s dtype, or fp32 work)
    with an fp32 result: the per-iteration body of the fused op, for the
    host-checked early exit (``NewtonConfig.fused_early_exit``; reference
    kernels/newton_slstm.py:2780-2922).  Not a registered op: the early exit
    synchronises with the host after every iteration."""
    batch, time, d_h = _slstm_shapes(wx, r)
    code = _validate("slstm_newton_step", wx, r, h0)
    cs32, bt, n_seq, h0 = _packed_args(cu_seqlens, block_table, wx, h0, d_h)
    if cs32 is None:
        h0 = _slstm_h0(h0, batch, d_h)
    if states.shape != (batch, time, 4, d_h):
        raise ValueError(f"states shape {tuple(states.shape)} != {(batch, time, 4, d_h)}")
    in_f32 = states.dtype == torch.float32
    if not in_f32 and states.dtype != wx.dtype:
        raise TypeError(f"slstm_newton_step: states dtype {states.dtype} is neither fp32 nor "
                        f"wx's {wx.dtype}")
    wx, r, states = wx.contiguous(), r.contiguous(), states.contiguous()
    out = torch.empty(batch, time, 4, d_h, dtype=torch.float32, device=wx.device)
    lib = _lib.load()
    _lib.sync_deterministic(lib)
    with torch.cuda.device(wx.device):
        if cs32 is None:
            nbytes = lib.prnn_slstm_newton_workspace_size(batch, time, d_h, 1, code)
            ws, tag = _slstm_workspace(nbytes, wx.device)
            rc = lib.prnn_slstm_newton_step(
                _ptr(wx), _ptr(r), _ptr(h0), _ptr(states), int(in_f32), _ptr(out), batch, time,
                d_h, float(omega), float(eps), code, _ptr(ws), ws.numel(), tag,
                _stream(wx.device),
            )
        else:
            nbytes = lib.prnn_slstm_newton_packed_workspace_size(time, d_h, 1, code)
            ws, tag = _slstm_workspace(nbytes, wx.device)
            rc = lib.prnn_slstm_newton_step_packed(
                _ptr(wx), _ptr(r), _ptr(h0), _ptr(states), int(in_f32), _ptr(out), time, d_h,
                float(omega), float(eps), code, _ptr(cs32), n_seq, _ptr(bt), _ptr(ws),
                ws.numel(), tag, _stream(wx.device),
            )
    _lib.check(rc, "slstm_newton_step")
    _check_lookback(ws, "slstm_newton_step")
    return out


def slstm_newton_eager(wx: Tensor, r: Tensor, h0: Tensor | None, states: Tensor, *,
                       omega: float, eps: float, cu_seqlens: Tensor | None = None,
                       block_table: Tensor | None = None) -> Tensor:
    """One Newton iteration with the reference's eager rounding
    (``scan_backend='eager'``, solvers/newton/__init__.py:516-543): the cell and
    its Jacobian rounded op by op in ``wx``'s dtype, the residual rounded, an
    fp32 scan, the rounded delta and the rounded update.  ``states`` and the
    result are in ``wx``'s dtype.  Not a registered op: the eager loop runs
    one launch per iteration from the host."""
    batch, time, d_h = _slstm_shapes(wx, r)
    code = _validate("slstm_newton_eager", wx, r, h0, states)
    cs32, bt, n_seq, h0 = _packed_args(cu_seqlens, block_table, wx, h0, d_h)
    if cs32 is None:
        h0 = _slstm_h0(h0, batch, d_h)
    if states.shape != (batch, time, 4, d_h):
        raise ValueError(f"states shape {tuple(states.shape)} != {(batch, time, 4, d_h)}")
    wx, r, states = wx.contiguous(), r.contiguous(), states.contiguous()
    out = torch.empty_like(states)
    lib = _lib.load()
    _lib.sync_deterministic(lib)
    with torch.cuda.device(wx.device):
        if cs32 is None:
            nbytes = lib.prnn_slstm_newton_workspace_size(batch, time, d_h, 1, code)
            ws, tag = _slstm_workspace(nbytes, wx.device)
            rc = lib.prnn_slstm_newton_eager(
                _ptr(wx), _ptr(r), _ptr(h0), _ptr(states), _ptr(out), batch, time, d_h,
                float(omega), float(eps), code, _ptr(ws), ws.numel(), tag, _stream(wx.device),
            )
        else:
            nbytes = lib.prnn_slstm_newton_packed_workspace_size(time, d_h, 1, code)
            ws, tag = _slstm_workspace(nbytes, wx.device)
            rc = lib.prnn_slstm_newton_eager_packed(
                _ptr(wx), _ptr(r), _ptr(h0), _ptr(states), _ptr(out), time, d_h, float(omega),
                float(eps), code, _ptr(cs32), n_seq, _ptr(bt), _ptr(ws), ws.numel(), tag,
                _stream(wx.device),
            )
    _lib.check(rc, "slstm_newton_eager")
    _check_lookback(ws, "slstm_newton_eager")
    return out


@newton_slstm_fused.register_fake
def _(wx, r, h0=None, states=None, block_table=None, cu_seqlens=None, *, max_iters, omega, eps,
      log_coords=False, scan_tile="assoc", time_loop=False, window_len=0):
    if states is not None:
        return torch.empty_like(states)
    batch, time, _ = wx.shape
    return wx.new_empty(batch, time, 4, r.shape[-1])


@torch.library.custom_op("pararnn::slstm_backward_fused", mutates_args=())
def slstm_backward_fused(
    wx: Tensor, r: Tensor, h0: Tensor | None, states: Tensor, grad: Tensor,
    cu_seqlens: Tensor | None = None, *, eps: float
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Eq. 2.6 backward of diag ParaSLSTM at ``H* = states`` on the GPU.

    Returns ``(g_wx, g_r, g_h0, g_b)``: ``dL/dwx`` ``(B, T, 4 d_h)`` in
    ``wx``'s dtype, ``g_r`` ``(4, d_h)`` fp32 (before the clamp mask on ``R``),
    ``g_h0 = J_0^T mu_0`` ``(B, 4, d_h)`` fp32 (zeros-input adjoint when ``h0``
    is None) and ``g_b = sum_{b,t} dL/dwx`` ``(4, d_h)`` fp32 (the ``W_x`` bias
    gradient, summed in the same pass).  The reference computes the same quantities with
    ``step_and_jacobian`` + ``reverse_scan_block4`` + ``slstm_recurrence_vjp``
    (solvers/newton/__init__.py:765-866, kernels/vjp_slstm.py:209-240).
    With ``cu_seqlens`` (a packed stream, ``B = 1``) nothing flows across a
    sequence head and ``g_h0`` is ``(S, 4, d_h)``, one row per sequence.
    """
    batch, time, d_h = _slstm_shapes(wx, r)
    code = _validate("slstm_backward_fused", wx, r, h0, states, grad)
    for name, t in (("states", states), ("grad", grad)):
        if t.shape != (batch, time, 4, d_h):
            raise ValueError(f"{name} shape {tuple(t.shape)} != {(batch, time, 4, d_h)}")
    wx, r, states, grad = wx.contiguous(), r.contiguous(), states.contiguous(), grad.contiguous()
    cs32, _, n_seq, h0 = _packed_args(cu_seqlens, None, wx, h0, d_h)
    if cs32 is None:
        h0 = _slstm_h0(h0, batch, d_h)
    g_wx = torch.empty_like(wx)
    g_r = torch.empty(4, d_h, dtype=torch.float32, device=wx.device)
    g_h0 = torch.zeros(n_seq if cs32 is not None else batch, 4, d_h, dtype=torch.float32,
                       device=wx.device)
    g_b = torch.empty(4, d_h, dtype=torch.float32, device=wx.device)
    lib = _lib.load()
    _lib.sync_deterministic(lib)
    with torch.cuda.device(wx.device):
        nbytes = lib.prnn_slstm_backward_workspace_size(batch, time, d_h, code)
        ws, tag = _slstm_workspace(nbytes, wx.device)
        if cs32 is None:
            rc = lib.prnn_slstm_backward_ex(
                _ptr(wx), _ptr(r), _ptr(h0), _ptr(states), _ptr(grad), _ptr(g_wx), _ptr(g_r),
                _ptr(g_h0), _ptr(g_b), batch, time, d_h, float(eps), code, _ptr(ws), ws.numel(),
                tag, _stream(wx.device),
            )
        else:
            rc = lib.prnn_slstm_backward_packed(
                _ptr(wx), _ptr(r), _ptr(h0), _ptr(states), _ptr(grad), _ptr(g_wx), _ptr(g_r),
                _ptr(g_h0), _ptr(g_b), time, d_h, float(eps), code, _ptr(cs32), n_seq,
                _ptr(ws), ws.numel(), tag, _stream(wx.device),
            )
    _lib.check(rc, "slstm_backward_fused")
    _check_lookback(ws, "slstm_backward_fused")
    return g_wx, g_r, g_h0, g_b


@slstm_backward_fused.register_fake
def _(wx, r, h0, states, grad, cu_seqlens=None, *, eps):
    batch, _, d_h = states.shape[0], states.shape[1], r.shape[-1]
    rows = batch if cu_seqlens is None else cu_seqlens.shape[0] - 1
    return (
        torch.empty_like(wx),
        wx.new_empty(4, d_h, dtype=torch.float32),
        wx.new_empty(rows, 4, d_h, dtype=torch.float32),
        wx.new_empty(4, d_h, dtype=torch.float32),
    )


# ---------------------------------------------------------------------------
# ParaGRU mix='head'
# ---------------------------------------------------------------------------


@torch.library.custom_op("pararnn::newton_gru_head_fused", mutates_args=())
def newton_gru_head_fused(
    wx: Tensor,
    a_z: Tensor,
    a_r: Tensor,
    a_n: Tensor,
    h0: Tensor | None = None,
    cu_seqlens: Tensor | None = None,
    *,
    max_iters: int,
    omega: float,
) -> Tensor:
    """Fused Alg. 1 for ``ParaGRU(mix='head')`` on the GPU (custom_ops.py:311-358).

    Initial guess ``f(h_prev0, x_t)`` (zeros except ``h0`` at t = 0), then
    ``max_iters`` Newton iterations, all in fp32; result in ``wx``'s dtype.
    ``cu_seqlens`` packs ``S`` sequences into ``wx`` ``(1, N, 3 d_h)`` with
    ``h0`` ``(S, d_h)``: the kernels cut the carry at every head (the
    reference's packed semantics, solvers/scan.py:206-216; its fused op takes
    rectangular batches only), or with ``PARARNN_AMD_PACKED=0`` the sequences
    run as padded length groups.
    """
    if a_z.dim() != 3 or a_z.shape[-1] != a_z.shape[-2]:
        raise ValueError(f"a_z needs (H,d,d), got {tuple(a_z.shape)}")
    n_heads, d_head, _ = a_z.shape
    if a_r.shape != a_z.shape or a_n.shape != a_z.shape:
        raise ValueError("a_z, a_r, a_n shape mismatch")
    d_h = n_heads * d_head
    if wx.dim() != 3 or wx.shape[-1] != 3 * d_h:
        raise ValueError(f"wx last dim {wx.shape[-1]} != 3 * d_h={3 * d_h}")
    if d_head > WIDE_MAX:
        raise TypeError(f"newton_gru_head_fused: pararnn_amd provides d_head <= {WIDE_MAX}, "
                        f"got {d_head}")
    if cu_seqlens is not None:
        from pararnn_amd.ragged import RaggedPlan, packed_in_kernel, validate_cu_seqlens

        if wx.shape[0] != 1:
            raise ValueError(f"cu_seqlens packs wx with batch=1, got batch={wx.shape[0]}")
        cs = validate_cu_seqlens(cu_seqlens, wx.shape[1], wx.device)
        n_seq = int(cs.numel()) - 1
        if h0 is not None and h0.shape != (n_seq, d_h):
            raise ValueError(f"h0 shape {tuple(h0.shape)} != {(n_seq, d_h)}")
        if packed_in_kernel():
            return _gru_head_dense(wx, a_z, a_r, a_n, h0, max_iters, omega, cs)
        plan = RaggedPlan(cs, wx.device)
        return plan.run(wx, h0, lambda w, h: _gru_head_dense(w, a_z, a_r, a_n, h, max_iters,
                                                              omega))
    return _gru_head_dense(wx, a_z, a_r, a_n, h0, max_iters, omega)


def _gru_head_dense(wx, a_z, a_r, a_n, h0, max_iters, omega, cs=None):
    """A rectangular batch, or (``cs``: checked int64 offsets) one packed stream."""
    n_heads, d_head, _ = a_z.shape
    d_h = n_heads * d_head
    batch, time, _ = wx.shape
    code = _validate("newton_gru_head_fused", wx, a_z, a_r, a_n, h0)
    rows = batch if cs is None else int(cs.numel()) - 1
    if h0 is not None and h0.shape != (rows, d_h):
        raise ValueError(f"h0 shape {tuple(h0.shape)} != {(rows, d_h)}")
    if max_iters < 0:
        raise ValueError(f"max_iters must be >= 0, got {max_iters!r}")
    if d_head > 64:
        return _gru_head_wide(wx, a_z, a_r, a_n, h0, int(max_iters), float(omega), code, cs)
    # heads narrower than 64 run as block-diagonal 64 x 64 blocks
    hb = HeadBlocks(n_heads, d_head, wx.device)
    wx = hb.to_blocks(wx, 3).contiguous()
    a_z, a_r, a_n = (hb.matrices(a) for a in (a_z, a_r, a_n))
    h0 = None if h0 is None else hb.to_blocks(h0).contiguous()
    out = wx.new_empty(batch, time, hb.d_pad)
    lib = _lib.load()
    with torch.cuda.device(wx.device):
        if cs is None:
            nbytes = lib.prnn_gru_head_newton_workspace_size(batch, time, hb.n_blocks, 64,
                                                             int(max_iters), code)
            ws = _workspace(nbytes, wx.device)
            rc = lib.prnn_gru_head_newton(
                _ptr(wx), _ptr(a_z), _ptr(a_r), _ptr(a_n), _ptr(h0), _ptr(out), batch, time,
                hb.n_blocks, 64, int(max_iters), float(omega), code, _ptr(ws), ws.numel(),
                _stream(wx.device),
            )
        else:
            cs32 = cs.to(device=wx.device, dtype=torch.int32).contiguous()
            nbytes = lib.prnn_gru_head_newton_packed_workspace_size(time, hb.n_blocks, 64,
                                                                    int(max_iters), code)
            ws = _workspace(nbytes, wx.device)
            rc = lib.prnn_gru_head_newton_packed(
                _ptr(wx), _ptr(a_z), _ptr(a_r), _ptr(a_n), _ptr(h0), _ptr(out), time,
                hb.n_blocks, 64, int(max_iters), float(omega), code, _ptr(cs32),
                int(cs32.numel()) - 1, None, _ptr(ws), ws.numel(), _stream(wx.device),
            )
    _lib.check(rc, "newton_gru_head_fused")
    return hb.from_blocks(out)


@newton_gru_head_fused.register_fake
def _(wx, a_z, a_r, a_n, h0=None, cu_seqlens=None, *, max_iters, omega):
    batch, time, _ = wx.shape
    return wx.new_empty(batch, time, int(a_z.shape[0] * a_z.shape[-1]))


@torch.library.custom_op("pararnn::gru_head_backward_fused", mutates_args=())
def gru_head_backward_fused(
    wx: Tensor, a_z: Tensor, a_r: Tensor, a_n: Tensor, h0: Tensor | None, states: Tensor,
    grad: Tensor, cu_seqlens: Tensor | None = None,
) -> tuple[Tensor, Tensor, Tensor]:
    """Eq. 2.6 backward of ``ParaGRU(mix='head')`` at ``H* = states`` on the GPU.

    Returns ``(g_wx, g_a, g_h0)``: ``dL/dwx`` ``(B, T, 3 d_h)`` in ``wx``'s
    dtype, ``g_a`` ``(3, H, d_head, d_head)`` fp32 (``dL/dA_z, dL/dA_r, dL/dA_n`` before
    clamp masks) and ``g_h0 = J_0^T mu_0`` ``(B, d_h)`` fp32 (zeros when ``h0`` is
    None).  The reference computes these with ``reverse_factor_scan_gru_head``,
    ``gru_head_t0_vjp`` and ``gru_head_recurrence_vjp``
    (solvers/newton/__init__.py:798-817, kernels/vjp_gru.py:656).
    ``cu_seqlens``: one packed stream ``(1, N, ...)`` of ``S`` sequences
    (nothing flows across a head; ``h0`` and ``g_h0`` are ``(S, d_h)``).
    """
    if a_z.dim() != 3 or a_z.shape[-1] != a_z.shape[-2]:
        raise ValueError(f"a_z needs (H,d,d), got {tuple(a_z.shape)}")
    n_heads, d_head, _ = a_z.shape
    if a_r.shape != a_z.shape or a_n.shape != a_z.shape:
        raise ValueError("a_z, a_r, a_n shape mismatch")
    if d_head > WIDE_MAX:
        raise TypeError(f"gru_head_backward_fused: pararnn_amd provides d_head <= {WIDE_MAX}, "
                        f"got {d_head}")
    d_h = n_heads * d_head
    if wx.dim() != 3 or wx.shape[-1] != 3 * d_h:
        raise ValueError(f"wx last dim {wx.shape[-1]} != 3 * d_h={3 * d_h}")
    batch, time, _ = wx.shape
    code = _validate("gru_head_backward_fused", wx, a_z, a_r, a_n, h0, states, grad)
    for name, t in (("states", states), ("grad", grad)):
        if t.shape != (batch, time, d_h):
            raise ValueError(f"{name} shape {tuple(t.shape)} != {(batch, time, d_h)}")
    cs32 = None
    rows = batch
    if cu_seqlens is not None:
        from pararnn_amd.ragged import validate_cu_seqlens

        if batch != 1:
            raise ValueError(f"cu_seqlens packs wx with batch=1, got batch={batch}")
        cs32 = validate_cu_seqlens(cu_seqlens, time, wx.device).to(torch.int32).contiguous()
        rows = int(cs32.numel()) - 1
    if h0 is not None and h0.shape != (rows, d_h):
        raise ValueError(f"h0 shape {tuple(h0.shape)} != {(rows, d_h)}")
    if d_head > 64:
        return _gru_head_wide_backward(wx, a_z, a_r, a_n, h0, states, grad, code, cs32)
    # heads narrower than 64 run as block-diagonal 64 x 64 blocks
    hb = HeadBlocks(n_heads, d_head, wx.device)
    wx = hb.to_blocks(wx, 3).contiguous()
    states = hb.to_blocks(states).contiguous()
    grad = hb.to_blocks(grad).contiguous()
    a_z, a_r, a_n = (hb.matrices(a) for a in (a_z, a_r, a_n))
    h0 = None if h0 is None else hb.to_blocks(h0).contiguous()
    g_wx = torch.empty_like(wx)
    g_a = torch.empty(3, hb.n_blocks, 64, 64, dtype=torch.float32, device=wx.device)
    g_h0 = torch.zeros(rows, hb.d_pad, dtype=torch.float32, device=wx.device)
    lib = _lib.load()
    with torch.cuda.device(wx.device):
        if cs32 is None:
            nbytes = lib.prnn_gru_head_backward_workspace_size(batch, time, hb.n_blocks, 64,
                                                               code)
            ws = _workspace(nbytes, wx.device)
            rc = lib.prnn_gru_head_backward(
                _ptr(wx), _ptr(a_z), _ptr(a_r), _ptr(a_n), _ptr(h0), _ptr(states), _ptr(grad),
                _ptr(g_wx), _ptr(g_a), _ptr(g_h0), batch, time, hb.n_blocks, 64, code,
                _ptr(ws), ws.numel(), _stream(wx.device),
            )
        else:
            nbytes = lib.prnn_gru_head_backward_packed_workspace_size(time, hb.n_blocks, 64,
                                                                      code)
            ws = _workspace(nbytes, wx.device)
            rc = lib.prnn_gru_head_backward_packed(
                _ptr(wx), _ptr(a_z), _ptr(a_r), _ptr(a_n), _ptr(h0), _ptr(states), _ptr(grad),
                _ptr(g_wx), _ptr(g_a), _ptr(g_h0), time, hb.n_blocks, 64, code, _ptr(cs32),
                rows, _ptr(ws), ws.numel(), _stream(wx.device),
            )
    _lib.check(rc, "gru_head_backward_fused")
    return hb.from_blocks(g_wx, 3), hb.head_grads(g_a), hb.from_blocks(g_h0)


@gru_head_backward_fused.register_fake
def _(wx, a_z, a_r, a_n, h0, states, grad, cu_seqlens=None):
    n_heads, d_head, _ = a_z.shape
    rows = states.shape[0] if cu_seqlens is None else cu_seqlens.shape[0] - 1
    return (
        torch.empty_like(wx),
        wx.new_empty(3, n_heads, d_head, d_head, dtype=torch.float32),
        wx.new_empty(rows, n_heads * d_head, dtype=torch.float32),
    )


# ---------------------------------------------------------------------------
# Wide heads, 64 < d_head <= 128 (the tier of the reference's streamed head
# kernel, kernels/newton_gru_head.py:121-150, 900-960)
# ---------------------------------------------------------------------------

WIDE_MAX = 128


def _wide_prev(states: Tensor, h0: Tensor | None, cs: Tensor | None) -> Tensor:
    """Previous state at every step (fp32): h0's row (zeros without h0) at each
    sequence's first step."""
    if cs is not None:
        from pararnn_amd.ragged import prepend_state_ragged

        return prepend_state_ragged(states, h0, cs)
    out = states.new_empty(states.shape)
    out[:, 1:] = states[:, :-1]
    out[:, 0] = 0 if h0 is None else h0
    return out


def _wide_gates(wx: Tensor, hp: Tensor, a: tuple[Tensor, Tensor, Tensor], code: int):
    """Gates ``z, r, n`` (fp32 ``(B, T, d)``) of every step from its previous
    state ``hp`` (fp32): ``sigmoid(wx_z + h A_z)``, ``sigmoid(wx_r + h A_r)``,
    ``tanh(wx_n + (h r) A_n)`` per head (cells/para_gru.py:414-467), in one
    HIP launch over all B*T rows (``prnn_gru_wide_gates``; ``wx`` and ``a`` in
    the storage dtype ``code``, contiguous).  Nothing here depends on the
    Newton walk, so it runs as wide parallel work before it."""
    batch, time, _ = wx.shape
    n_heads, d_head, _ = a[0].shape
    shape = (batch, time, n_heads * d_head)
    z, r, n = (torch.empty(shape, dtype=torch.float32, device=wx.device) for _ in range(3))
    lib = _lib.load()
    with torch.cuda.device(wx.device):
        rc = lib.prnn_gru_wide_gates(
            _ptr(wx), _ptr(hp), _ptr(a[0]), _ptr(a[1]), _ptr(a[2]), _ptr(z), _ptr(r), _ptr(n),
            batch * time, n_heads, d_head, code, _stream(wx.device),
        )
    _lib.check(rc, "gru head gates (wide heads)")
    return z, r, n


def _wide_guess(wx: Tensor, a: tuple[Tensor, Tensor, Tensor], h0: Tensor | None,
                cs: Tensor | None, code: int) -> Tensor:
    """The initial guess ``f(h_prev0, x)`` (fp32), ``h_prev0 = 0`` except h0's
    row at each sequence's first step (reference solvers/newton/__init__.py:
    925-940).  With a zero previous state the cell is elementwise, ``lerp(0,
    tanh(wx_n), sigmoid(wx_z))``; only the first steps with h0 need the gate
    mat-vecs (``prnn_gru_wide_gates`` on those rows alone)."""
    batch, time, three_d = wx.shape
    d_h = three_d // 3
    z = torch.sigmoid(wx[..., :d_h].float())
    n = torch.tanh(wx[..., 2 * d_h:].float())
    states = torch.lerp(torch.zeros_like(n), n, z)
    if h0 is not None:
        if cs is None:
            bi = torch.arange(batch, device=wx.device)
            ti = torch.zeros(batch, dtype=torch.long, device=wx.device)
        else:
            ti = cs[:-1].to(device=wx.device, dtype=torch.long)
            bi = torch.zeros_like(ti)
        hp = h0.unsqueeze(0).contiguous()
        zs, _, ns = _wide_gates(wx[bi, ti].unsqueeze(0).contiguous(), hp, a, code)
        states[bi, ti] = torch.lerp(hp, ns, zs)[0]
    return states


def _wide_workspace_cap(dev: torch.device) -> int:
    """Largest one-launch workspace the wide tier takes (a quarter of the
    device's memory: 8 bytes per element for each of K - 1 iterates and six
    gate planes); larger solves run one launch per iteration instead, whose
    buffers are a few fp32 copies of the states."""
    return torch.cuda.get_device_properties(dev).total_memory // 4


def _gru_head_wide(wx, a_z, a_r, a_n, h0, max_iters, omega, code, cs=None):
    """Forward of the wide tier: the initial guess ``f(h_prev0, x)``, then the
    Newton iterations.  K >= 2: one launch (``prnn_gru_wide_newton``) in which,
    per (iteration, sequence, head), gate workgroups feed a walk, the
    iterations a few blocks of steps apart
    (``PARARNN_AMD_WIDE_FUSED=0``: one launch per iteration, as for K = 1).
    K = 1 (and solves whose one-launch workspace exceeds ``_wide_workspace_cap``):
    the gates at the iterate (``prnn_gru_wide_gates``) and one HIP walk per
    (sequence, head) for ``delta`` and the update (``prnn_gru_wide_walk``), per
    iteration.  fp32 work; the result in ``wx``'s dtype."""
    n_heads, d_head, _ = a_z.shape
    batch, time, _ = wx.shape
    d_h = n_heads * d_head
    wx_c = wx.contiguous()
    a_k = tuple(t.contiguous() for t in (a_z, a_r, a_n))
    h0_32 = None if h0 is None else h0.float()
    states = _wide_guess(wx_c, a_k, h0_32, cs, code)
    if max_iters == 0:
        return states.to(wx.dtype)
    cs32 = None if cs is None else cs.to(device=wx.device, dtype=torch.int32).contiguous()
    n_seq = 0 if cs32 is None else int(cs32.numel()) - 1
    lib = _lib.load()
    nbytes = lib.prnn_gru_wide_newton_workspace_size(batch, time, n_heads, d_head, max_iters)
    if (max_iters >= 2 and os.environ.get("PARARNN_AMD_WIDE_FUSED", "1") != "0"
            and nbytes <= _wide_workspace_cap(wx.device)):
        # all iterations in one launch, each a few blocks behind the last
        out = wx.new_empty(batch, time, d_h)
        ws, tag = _slstm_workspace(nbytes, wx.device)
        h0_c = None if h0_32 is None else h0_32.contiguous()
        guess = states.contiguous()
        with torch.cuda.device(wx.device):
            rc = lib.prnn_gru_wide_newton(
                _ptr(wx_c), _ptr(a_k[0]), _ptr(a_k[1]), _ptr(a_k[2]), _ptr(h0_c), _ptr(guess),
                _ptr(out), batch, time, n_heads, d_head, max_iters, float(omega), code,
                _ptr(cs32), n_seq, _ptr(ws), ws.numel(), tag, _stream(wx.device),
            )
        _lib.check(rc, "newton_gru_head_fused (wide heads)")
        _check_lookback(ws, "newton_gru_head_fused (wide heads)")
        return out
    out = None
    for it in range(max_iters):
        hp = _wide_prev(states, h0_32, cs).contiguous()
        z, r, n = _wide_gates(wx_c, hp, a_k, code)
        last = it == max_iters - 1
        narrow = last and wx.dtype != torch.float32
        out = wx.new_empty(batch, time, d_h) if narrow else states
        with torch.cuda.device(wx.device):
            rc = lib.prnn_gru_wide_walk(
                _ptr(z), _ptr(r), _ptr(n), _ptr(hp), _ptr(states), _ptr(a_k[0]), _ptr(a_k[1]),
                _ptr(a_k[2]), _ptr(out), int(not narrow), batch, time, n_heads, d_head,
                float(omega), code, _ptr(cs32), n_seq, _stream(wx.device),
            )
        _lib.check(rc, "newton_gru_head_fused (wide heads)")
        states = out
    return out if out.dtype == wx.dtype else out.to(wx.dtype)


def _gru_head_wide_backward(wx, a_z, a_r, a_n, h0, states, grad, code, cs32=None):
    """Eq. 2.6 backward of the wide tier at ``H* = states``: the gates at H*
    (``prnn_gru_wide_gates``), one HIP adjoint walk per (sequence, head)
    (``prnn_gru_wide_reverse``: dL/dwx and dL/dh0), then dL/dA as GEMMs over
    the B*T rows, ``sum_t X_t^T D_t`` with X = h_prev (z, r) or h_prev r (n)."""
    n_heads, d_head, _ = a_z.shape
    batch, time, _ = wx.shape
    d_h = n_heads * d_head
    cs = None if cs32 is None else cs32.long()
    rows = batch if cs32 is None else int(cs32.numel()) - 1
    a_k = tuple(t.contiguous() for t in (a_z, a_r, a_n))
    hp = _wide_prev(states.float(), None if h0 is None else h0.float(), cs).contiguous()
    z, r, n = _wide_gates(wx.contiguous(), hp, a_k, code)
    grad = grad.contiguous()
    g_wx = torch.empty(batch, time, 3 * d_h, dtype=torch.float32, device=wx.device)
    g_h0 = torch.zeros(rows, d_h, dtype=torch.float32, device=wx.device)
    lib = _lib.load()
    with torch.cuda.device(wx.device):
        rc = lib.prnn_gru_wide_reverse(
            _ptr(z), _ptr(r), _ptr(n), _ptr(hp), _ptr(grad), int(grad.dtype == torch.float32),
            _ptr(a_k[0]), _ptr(a_k[1]), _ptr(a_k[2]), _ptr(g_wx), _ptr(g_h0), batch, time,
            n_heads, d_head, code, _ptr(cs32), 0 if cs32 is None else rows, _stream(wx.device),
        )
    _lib.check(rc, "gru_head_backward_fused (wide heads)")
    n_rows = batch * time
    dpre = g_wx.view(n_rows, 3, n_heads, d_head).permute(1, 2, 0, 3)  # (3, H, rows, dh)
    xs = hp.view(n_rows, n_heads, d_head).transpose(0, 1)  # (H, rows, dh)
    xr = (hp * r).view(n_rows, n_heads, d_head).transpose(0, 1)
    g_a = torch.stack([torch.bmm(x.transpose(1, 2), dpre[g])
                       for g, x in enumerate((xs, xs, xr))])
    return g_wx.to(wx.dtype), g_a, g_h0
