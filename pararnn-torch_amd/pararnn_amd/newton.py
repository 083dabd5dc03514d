"""``newton_apply``: the reference's Newton + scan entry point over the HIP kernels.

Control flow follows the reference (``solvers/newton/__init__.py:212-324,
347-441, 582-693``, ``solvers/newton/dispatch.py:71-227``,
``solvers/newton/picard.py:22-186``, ``kernels/fused_newton.py:29-389``):

* ``max_iters=None`` resolves K from ``newton_iters_by_t`` or the library K;
* ``picard_iters=None`` resolves the ParaSLSTM Picard depth from T (1/3/5) and
  turns on the adaptive retry, which re-solves at the next depth when the
  residual exceeds ``picard_retry_atol``;
* ``scan_backend`` 'auto' / 'fused' select the HIP kernels for
  ``ParaSLSTM(mix='diag')`` and ``ParaGRU(mix='head')`` on a ROCm device;
  'eager' runs the reference's eager loop on the GPU (the sLSTM iterations in
  a kernel that rounds like the eager tensor ops);
* after the solve the residual gate re-evaluates ``max |F|`` with the cell's
  torch ``step`` and raises :class:`NewtonDivergenceError` above
  ``residual_fail``.

The Newton solve itself never runs on the CPU: inputs on another device, or
backends this build does not provide ('triton', 'context_parallel'), raise
instead of falling back.
"""

from __future__ import annotations

import contextlib
import logging
import math
import os
from collections.abc import Iterator
from dataclasses import replace

import torch
from torch import Tensor, nn

from pararnn_amd import determinism, ops
from pararnn_amd.cells import SLSTM_HIDDEN, ParaGRU, ParaSLSTM
from pararnn_amd.ragged import (
    RaggedPlan,
    gather_h0,
    packed_in_kernel,
    prepend_state_ragged,
    validate_cu_seqlens,
)
from pararnn_amd.config import (
    _RESIDUAL_WARN,
    LIBRARY_NEWTON_ITERS,
    NewtonConfig,
    NewtonDivergenceError,
    NewtonStats,
    lookup_iters_by_t,
    validate_config,
)

log = logging.getLogger("pararnn_amd.newton")

_PICARD_RUNGS = (1, 3, 5)


def slstm_auto_picard(seq_len: int) -> int:
    """Picard depth by T: 1 if T <= 64, 3 if T <= 2048, else 5 (picard.py:22-45)."""
    t = int(seq_len)
    return 1 if t <= 64 else (3 if t <= 2048 else 5)


def slstm_picard_next(picard_iters: int) -> int | None:
    """Next rung of the 1 -> 3 -> 5 ladder, or None at the top (picard.py:48-68)."""
    p = int(picard_iters)
    for rung in _PICARD_RUNGS:
        if p < rung:
            return rung
    return None


def auto_newton_iters(cell: nn.Module, seq_len: int, *, schedule=None) -> int:
    """K when ``max_iters=None``: the pinned table, else the library K (k_star.py:89-118)."""
    if schedule is not None:
        if callable(schedule):
            return int(schedule(int(seq_len)))
        return lookup_iters_by_t(schedule, int(seq_len))
    return int(LIBRARY_NEWTON_ITERS)


def _fusable(cell: nn.Module, x: Tensor) -> bool:
    if x.device.type != "cuda" or x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        return False
    if isinstance(cell, ParaSLSTM):
        return cell.mix == "diag"
    if isinstance(cell, ParaGRU):
        return cell.mix == "head" and cell.d_head <= 128
    return False


def _fused_error(cell: nn.Module, x: Tensor) -> str:
    return (
        "pararnn_amd's Newton solve ('fused' / 'auto' / 'eager') needs ParaSLSTM(mix='diag') or "
        "ParaGRU(mix='head', d_head <= 128) on a ROCm GPU in float32/bfloat16/float16 "
        f"(got {type(cell).__name__}(mix={getattr(cell, 'mix', None)!r}) "
        f"{x.dtype} on {x.device})"
    )


def _resolve_picard(cell: nn.Module, x: Tensor, config: NewtonConfig) -> NewtonConfig:
    if config.picard_iters is None:
        if isinstance(cell, ParaSLSTM):
            return replace(config, picard_iters=slstm_auto_picard(x.shape[1]))
        return replace(config, picard_iters=0)
    if config.picard_iters and not isinstance(cell, ParaSLSTM):
        raise TypeError(
            f"NewtonConfig(picard_iters=) is ParaSLSTM only (got {type(cell).__name__})"
        )
    return config


def _resolve_backend(cell: nn.Module, x: Tensor, config: NewtonConfig) -> NewtonConfig:
    auto_p = config.picard_iters is None
    config = _resolve_picard(cell, x, config)
    if config.picard_adapt is None:
        config = replace(config, picard_adapt=auto_p and isinstance(cell, ParaSLSTM))
    requested = config.scan_backend
    if config.coords == "log":
        raise TypeError("NewtonConfig(coords='log') is not provided by pararnn_amd")
    if requested in ("triton", "context_parallel"):
        raise NotImplementedError(
            f"scan_backend={requested!r} is not provided by pararnn_amd; its Newton solve "
            "runs the HIP kernels ('fused' / 'auto', or 'eager' for the eager rounding)"
        )
    if not _fusable(cell, x):
        raise TypeError(_fused_error(cell, x))
    if requested == "eager":
        return config
    return replace(config, scan_backend="fused")


def _prepend(states: Tensor, h0: Tensor | None) -> Tensor:
    """Previous state at every t: h0 (or zeros) then states[:, :-1] (layout.py:78-90)."""
    out = states.new_empty(states.shape)
    if h0 is None:
        out[:, 0] = 0
    else:
        out[:, 0] = h0
    out[:, 1:] = states[:, :-1]
    return out


def fused_newton(
    cell: nn.Module,
    wx: Tensor,
    *,
    max_iters: int,
    omega: float,
    h0: Tensor | None,
    log_coords: bool = False,
    picard_iters: int = 0,
    scan_tile: str = "assoc",
    fused_time_loop: bool = False,
    fused_window_len: int | None = None,
    cu_seqlens: Tensor | None = None,
    block_table: Tensor | None = None,
) -> Tensor:
    """Run the fused Alg. 1 for a supported cell (kernels/fused_newton.py:29-389)."""
    if isinstance(cell, ParaGRU) and cell.mix == "head":
        if log_coords:
            raise TypeError("fused log coords is ParaSLSTM only")
        if picard_iters:
            raise TypeError("fused Picard is ParaSLSTM only")
        if scan_tile != "assoc":
            raise TypeError("fused scan_tile is ParaSLSTM only")
        if fused_time_loop:
            raise TypeError("fused_time_loop is ParaSLSTM only")
        if block_table is not None:
            # paged h0: the rows the table names (one per sequence, or batch row)
            rows = wx.shape[0] if cu_seqlens is None else int(cu_seqlens.numel()) - 1
            h0 = gather_h0(h0, block_table, rows, (int(cell.d_h),))
        a_z, a_r, a_n = cell.clipped_a_head()
        return ops.newton_gru_head_fused(
            wx, a_z, a_r, a_n, h0, cu_seqlens, max_iters=max_iters, omega=omega
        )
    if isinstance(cell, ParaSLSTM) and cell.mix == "diag":
        if cu_seqlens is not None and not packed_in_kernel():
            # packed sequences as padded length groups, each from its own h0
            if block_table is not None:
                h0 = gather_h0(h0, block_table, int(cu_seqlens.numel()) - 1,
                               (4, int(cell.d_h)))
            plan = RaggedPlan(validate_cu_seqlens(cu_seqlens, wx.shape[1]), wx.device)
            return plan.run(wx, h0, lambda w, h: fused_newton(
                cell, w, max_iters=max_iters, omega=omega, h0=h,
                log_coords=log_coords, picard_iters=picard_iters, scan_tile=scan_tile,
                fused_time_loop=fused_time_loop, fused_window_len=fused_window_len))
        if block_table is not None and cu_seqlens is None:
            # paged h0 of a rectangular batch: the B rows the table names
            h0 = gather_h0(h0, block_table, wx.shape[0], (4, int(cell.d_h)))
            block_table = None
        # packed streams run in the kernels themselves: heads cut the carry and
        # read their h0 row (block_table[s] of a pool when given)
        r = cell.clipped_r()
        states = ops.slstm_init_fused(wx, r, h0, cu_seqlens, block_table,
                                      picard_iters=int(picard_iters), eps=cell.eps)
        return ops.newton_slstm_fused(
            wx, r, h0, states, block_table, cu_seqlens,
            max_iters=max_iters, omega=omega, eps=cell.eps, log_coords=log_coords,
            scan_tile=scan_tile, time_loop=fused_time_loop,
            window_len=0 if fused_window_len is None else int(fused_window_len),
        )
    raise TypeError(_fused_error(cell, wx))


def _prepend_any(states: Tensor, h0: Tensor | None, cu_seqlens: Tensor | None) -> Tensor:
    if cu_seqlens is None:
        return _prepend(states, h0)
    return prepend_state_ragged(states, h0, cu_seqlens)


def _fill_stats(cell, x, states, h0, config, *, iters, stats, history=(), known=None,
                cu_seqlens=None) -> None:
    """Residual gate (newton/__init__.py:582-636): one extra cell step over T."""
    if stats is None and config.residual_fail is None:
        return
    if known is None:
        pred = cell.step(_prepend_any(states, h0, cu_seqlens), x)
        res = float((pred - states).detach().abs().amax())
    else:
        res = known
    hist = tuple(history)
    if stats is not None:
        stats.max_residual = res
        stats.iters = iters
        stats.scan_backend = config.scan_backend
        stats.picard_iters = int(config.picard_iters or 0)
        stats.residual_history = hist
    cap = config.residual_fail
    diverged = not math.isfinite(res) or (cap is not None and res > cap)
    if diverged and cap is not None:
        raise NewtonDivergenceError(
            f"Newton residual {res:.3e} after {iters} iters exceeds residual_fail="
            f"{cap:g} (seq_len={x.shape[1]}, picard={int(config.picard_iters or 0)}, "
            f"history={hist[-8:]!r}). For ParaSLSTM raise picard_iters."
        )
    if res > _RESIDUAL_WARN and log.isEnabledFor(logging.WARNING):
        log.warning("newton_residual_high max_residual=%g iters=%d", res, iters)


def _newton_solve(cell, x, config, *, h0, stats, wx=None, cu_seqlens=None,
                  block_table=None) -> Tensor:
    if config.chunk_len is not None:
        return _newton_chunked(cell, x, config, h0=h0, stats=stats)
    if wx is None:
        wx = cell.W_x(x)
    gate_h0 = h0 if block_table is None else gather_h0(
        h0, block_table, int(cu_seqlens.numel()) - 1, _state_tail(cell))
    if config.scan_backend == "eager":
        states, iters, history, last, current = _newton_eager(cell, wx, config, h0=h0,
                                                              cu_seqlens=cu_seqlens)
        if not torch.compiler.is_compiling():
            _fill_stats(cell, x, states, h0, config, iters=iters, stats=stats, history=history,
                        known=last if current else None, cu_seqlens=cu_seqlens)
        return states
    if config.fused_early_exit and not torch.compiler.is_compiling():
        states, iters, history = _fused_early_exit(cell, wx, config, h0=h0,
                                                   cu_seqlens=cu_seqlens,
                                                   block_table=block_table)
        _fill_stats(cell, x, states, gate_h0, config, iters=iters, stats=stats, history=history,
                    known=history[-1] if history else float("nan"), cu_seqlens=cu_seqlens)
        return states
    states = fused_newton(
        cell, wx,
        max_iters=int(config.max_iters), omega=float(config.omega), h0=h0,
        log_coords=config.coords == "log", picard_iters=int(config.picard_iters or 0),
        scan_tile=config.scan_tile, fused_time_loop=config.fused_time_loop,
        fused_window_len=config.fused_window_len, cu_seqlens=cu_seqlens,
        block_table=block_table,
    )
    if not torch.compiler.is_compiling():
        _fill_stats(cell, x, states, gate_h0, config, iters=int(config.max_iters), stats=stats,
                    cu_seqlens=cu_seqlens)
    return states


def _fused_early_exit(cell, wx, config, *, h0, cu_seqlens=None,
                      block_table=None) -> tuple[Tensor, int, list[float]]:
    """``NewtonConfig.fused_early_exit`` (newton/__init__.py:696-762, the early-exit
    branch of kernels/newton_slstm.py:2892-2922): the fused iterations one at a
    time on the fp32 work iterate; after each, the host reads max|F| of the
    iterate rounded to ``wx``'s dtype and stops below ``residual_atol``.
    Returns ``(states, iterations run, residual history)``.  ParaSLSTM
    mix='diag' only, as in the reference."""
    if not (isinstance(cell, ParaSLSTM) and cell.mix == "diag"):
        raise TypeError("fused_early_exit is mix='diag' only; ParaGRU(mix='head') uses fixed K")
    atol = float(config.residual_atol)
    r = cell.clipped_r()
    P = int(config.picard_iters or 0)
    work = ops.slstm_init_fused(wx, r, h0, cu_seqlens, block_table, picard_iters=P, eps=cell.eps)
    gate_h0 = h0 if block_table is None else gather_h0(
        h0, block_table, int(cu_seqlens.numel()) - 1, _state_tail(cell))
    history: list[float] = []
    states = work
    for it in range(int(config.max_iters)):
        work = ops.slstm_newton_step(wx, r, h0, work, omega=float(config.omega), eps=cell.eps,
                                     cu_seqlens=cu_seqlens, block_table=block_table)
        states = work.to(wx.dtype)
        pred = cell.step(_prepend_any(states, gate_h0, cu_seqlens), None, wx=wx)
        res = float((pred - states).abs().amax())
        history.append(res)
        if res < atol:
            return states, it + 1, history
    return states, int(config.max_iters), history


def _newton_eager(cell, wx, config, *, h0, cu_seqlens=None):
    """``scan_backend='eager'``: the reference's eager Newton loop
    (newton/__init__.py:467-549) on the GPU.  Returns ``(states, iterations,
    residual history, last residual, whether it is the residual of states)``.

    ParaSLSTM diag: the Picard guess (the same warm start as the fused path:
    the reference's eager and fused paths share it, picard.py:161-186), then
    one launch per iteration whose cell, Jacobian, residual, delta and update
    round in the tensor dtype where the eager tensor ops round
    (``prnn_slstm_newton_eager``).  ParaGRU head: the fused kernels (fp32 work
    on the tensor dtype), since its eager and fused semantics agree to within
    the bf16 tolerance.  With ``residual_atol`` set (and not compiling) the
    host reads max|F| of the current iterate before each update and stops
    below it, as the eager loop does; that iteration counts."""
    atol = config.residual_atol if not torch.compiler.is_compiling() else None
    K = int(config.max_iters)
    omega = float(config.omega)
    history: list[float] = []

    def residual(states: Tensor) -> float:
        pred = cell.step(_prepend_any(states, h0, cu_seqlens), None, wx=wx)
        return float((pred - states).abs().amax())

    if isinstance(cell, ParaSLSTM):
        r = cell.clipped_r()
        states = ops.slstm_init_fused(wx, r, h0, cu_seqlens, None,
                                      picard_iters=int(config.picard_iters or 0), eps=cell.eps)
        for it in range(K):
            if atol is not None:
                history.append(residual(states))
                if history[-1] < atol:
                    return states, it + 1, history, history[-1], True
            states = ops.slstm_newton_eager(wx, r, h0, states, omega=omega, eps=cell.eps,
                                            cu_seqlens=cu_seqlens)
        return states, K, history, (history[-1] if history else float("nan")), False

    def solve(k: int) -> Tensor:
        return fused_newton(cell, wx, max_iters=k, omega=omega, h0=h0, cu_seqlens=cu_seqlens)

    if atol is None:
        return solve(K), K, history, float("nan"), False
    # the iterate before update `it` is the K = it fused solve
    for it in range(K):
        states = solve(it)
        history.append(residual(states))
        if history[-1] < atol:
            return states, it + 1, history, history[-1], True
    return solve(K), K, history, history[-1] if history else float("nan"), False


def _newton_chunked(cell, x, config, *, h0, stats) -> Tensor:
    """Newton on windows of ``chunk_len``; each window's last state seeds the next
    (newton/__init__.py:552-579)."""
    length = int(config.chunk_len)
    inner = replace(config, chunk_len=None)
    parts = []
    carry = h0
    iters = 0
    for t0 in range(0, x.shape[1], length):
        st = NewtonStats() if stats is not None else None
        piece = _newton_forward(cell, x[:, t0:t0 + length], inner, h0=carry, stats=st)
        parts.append(piece)
        carry = piece[:, -1]
        if st is not None:
            iters += st.iters
    states = torch.cat(parts, dim=1)
    _fill_stats(cell, x, states, h0, config, iters=iters, stats=stats)
    return states


def _picard_retry_needed(res: float, config: NewtonConfig) -> bool:
    if not math.isfinite(res):
        return True
    cap = config.picard_retry_atol
    if cap is not None and res > cap:
        return True
    fail = config.residual_fail
    return fail is not None and res > fail


def _newton_forward(cell, x, config, *, h0, stats, wx=None, cu_seqlens=None,
                    block_table=None) -> Tensor:
    """The solve; ``wx`` (unchunked only) reuses a projection already computed.
    ``cu_seqlens`` / ``block_table``: a packed diag-sLSTM stream solved in the
    kernels."""
    if config.chunk_len is not None:
        return _newton_chunked(cell, x, config, h0=h0, stats=stats)
    packed = dict(cu_seqlens=cu_seqlens, block_table=block_table)
    if not (config.picard_adapt and isinstance(cell, ParaSLSTM)) or torch.compiler.is_compiling():
        return _newton_solve(cell, x, config, h0=h0, stats=stats, wx=wx, **packed)
    # Adaptive Picard ladder (picard.py:105-158).
    cfg = config
    while True:
        st = stats if stats is not None else NewtonStats()
        states = _newton_solve(cell, x, replace(cfg, residual_fail=None), h0=h0, stats=st,
                               wx=wx, **packed)
        res = st.max_residual
        nxt = slstm_picard_next(int(cfg.picard_iters or 0))
        if _picard_retry_needed(res, config) and nxt is not None:
            log.info("picard_adapt from_p=%d to_p=%d max_residual=%g",
                     int(cfg.picard_iters or 0), nxt, res)
            cfg = replace(cfg, picard_iters=nxt)
            continue
        cap = config.residual_fail
        if cap is not None and (not math.isfinite(res) or res > cap):
            _fill_stats(cell, x, states, h0, config, iters=st.iters, stats=st,
                        history=st.residual_history, known=res, cu_seqlens=cu_seqlens)
        return states


def newton_apply(
    cell: nn.Module,
    x: Tensor,
    config: NewtonConfig | None = None,
    *,
    h0: Tensor | None = None,
    stats: NewtonStats | None = None,
    cu_seqlens: Tensor | None = None,
    block_table: Tensor | None = None,
) -> Tensor:
    """Solve ``F(H) = 0`` with Newton + parallel scan on the GPU (newton/__init__.py:212-324).

    Parameters and returns as in the reference: ``x`` ``(B, T, d_in)``;
    ``H`` ``(B, T, 4, d_h)`` for ParaSLSTM, ``(B, T, d_h)`` for ParaGRU.
    """
    config = config or NewtonConfig()
    validate_config(config)
    if config.max_iters is None:
        config = replace(
            config,
            max_iters=auto_newton_iters(cell, x.shape[1], schedule=config.newton_iters_by_t),
        )
    if cu_seqlens is not None:
        _check_ragged_args(x, config)
    config = _resolve_backend(cell, x, config)
    params = tuple(cell.parameters())
    needs_grad = torch.is_grad_enabled() and (
        x.requires_grad
        or (h0 is not None and h0.requires_grad)
        or any(p.requires_grad for p in params)
    )
    if block_table is not None:
        if config.scan_backend != "fused":
            raise ValueError("block_table newton needs scan_backend='fused' (or auto on a ROCm "
                             "GPU)")
        if config.chunk_len is not None:
            raise ValueError("block_table cannot be combined with chunk_len")
        if needs_grad:
            raise RuntimeError("block_table newton is inference-only")
    with _newton_precision_region(x.device):
        if cu_seqlens is not None:
            if _packable(cell) and packed_in_kernel():
                return _newton_packed(cell, x, config, h0=h0, stats=stats,
                                      cu_seqlens=cu_seqlens, block_table=block_table,
                                      needs_grad=needs_grad)
            return _newton_ragged(cell, x, config, h0=h0, stats=stats, cu_seqlens=cu_seqlens,
                                  block_table=block_table, needs_grad=needs_grad)
        if block_table is not None:
            h0 = gather_h0(h0, block_table, x.shape[0], _state_tail(cell))
        if not needs_grad:
            return _newton_forward(cell, x, config, h0=h0, stats=stats)
        has_h0 = h0 is not None
        h0_leaf = h0 if has_h0 else x.new_zeros(())
        _fwd_pack.clear()
        _fwd_pack.update(cell=cell, config=config, stats=stats, has_h0=has_h0)
        try:
            return _NewtonFixedPoint.apply(x, h0_leaf, *params)
        finally:
            _fwd_pack.clear()


@contextlib.contextmanager
def _newton_precision_region(device: torch.device) -> Iterator[None]:
    """Keep the solve and the eq. 2.6 backward in the tensors' dtype under an
    outer ``autocast`` (newton/__init__.py:193-209): AMP would round ``W_x(x)``
    while the states stay in the module dtype.  Callers that want bf16 Newton
    put the module and ``x`` in bf16."""
    if device.type in ("cuda", "cpu") and torch.is_autocast_enabled(device.type):
        with torch.autocast(device_type=device.type, enabled=False):
            yield
        return
    yield


def _state_tail(cell: nn.Module) -> tuple[int, ...]:
    slots = getattr(cell, "state_slots", 1)
    return (int(cell.d_h),) if slots == 1 else (int(slots), int(cell.d_h))


def _check_ragged_args(x: Tensor, config: NewtonConfig) -> None:
    if x.shape[0] != 1:
        raise ValueError(f"cu_seqlens packs x with batch=1, got batch={x.shape[0]}")
    if config.chunk_len is not None:
        raise ValueError("chunk_len cannot be combined with cu_seqlens")
    if config.fused_time_loop:
        raise ValueError("fused_time_loop cannot be combined with cu_seqlens")


def _packable(cell: nn.Module) -> bool:
    """Cells whose kernels solve packed streams in place."""
    return (isinstance(cell, ParaSLSTM) and cell.mix == "diag") or (
        isinstance(cell, ParaGRU) and cell.mix == "head")


def _newton_packed(cell, x, config, *, h0, stats, cu_seqlens, block_table, needs_grad):
    """A packed stream in one solve (diag sLSTM, head GRU): the kernels cut the
    carry at every sequence head and read each head's h0 row themselves
    (block_table rows of a pool when given: in the sLSTM kernels, gathered
    first for the head GRU), as the reference's packed semantics
    (solvers/scan.py:206-216, layout.py:115-138); K, P, the Picard ladder and
    the residual gate act on the packed stream (newton/__init__.py:327-355)."""
    cs = validate_cu_seqlens(cu_seqlens, x.shape[1], x.device)
    n_seq = int(cs.numel()) - 1
    if block_table is None and h0 is not None and h0.shape[0] != n_seq:
        raise ValueError(f"h0 batch {h0.shape[0]} != n_seq {n_seq}")
    if not needs_grad:
        return _newton_forward(cell, x, config, h0=h0, stats=stats, cu_seqlens=cs,
                               block_table=block_table)
    has_h0 = h0 is not None
    h0_leaf = h0 if has_h0 else x.new_zeros(())
    _fwd_pack.clear()
    _fwd_pack.update(cell=cell, config=config, stats=stats, has_h0=has_h0, cu_seqlens=cs)
    try:
        return _NewtonFixedPoint.apply(x, h0_leaf, *tuple(cell.parameters()))
    finally:
        _fwd_pack.clear()


def _newton_ragged(cell, x, config, *, h0, stats, cu_seqlens, block_table, needs_grad):
    """Packed sequences (``cu_seqlens``) as a padded batch through the same solve
    (newton/__init__.py:327-355 for the validation).  K, P and the Picard ladder
    are resolved on the packed stream, and the residual gate is evaluated on the
    packed result with the ragged prepend (h0[s] at each head)."""
    cs = validate_cu_seqlens(cu_seqlens, x.shape[1])
    n_seq = int(cs.numel()) - 1
    if block_table is not None:
        h0 = gather_h0(h0, block_table, n_seq, _state_tail(cell))
    elif h0 is not None and h0.shape[0] != n_seq:
        raise ValueError(f"h0 batch {h0.shape[0]} != n_seq {n_seq}")
    if config.fused_early_exit:
        if not (isinstance(cell, ParaSLSTM) and cell.mix == "diag"):
            raise TypeError("fused_early_exit is mix='diag' only; ParaGRU(mix='head') uses "
                            "fixed K")
        # an exit decided per length group would not be the packed stream's
        raise ValueError("fused_early_exit with cu_seqlens runs in the packed kernels; it is "
                         "not available with PARARNN_AMD_PACKED=0 (length groups)")
    plan = RaggedPlan(cs, x.device)
    ladder = bool(config.picard_adapt) and isinstance(cell, ParaSLSTM)
    inner = replace(config, picard_adapt=False, residual_fail=None)
    hist = []
    while True:
        if needs_grad:
            states = plan.run(x, h0, lambda xp, h: newton_apply(cell, xp, inner, h0=h))
        else:
            states = plan.run(x, h0, lambda xp, h: _newton_forward(cell, xp, inner, h0=h,
                                                                  stats=None))
        if stats is None and config.residual_fail is None and not ladder:
            return states
        with torch.no_grad():
            pred = cell.step(prepend_state_ragged(states.detach(), h0, cs), x.detach())
            res = float((pred - states.detach()).abs().amax())
        hist.append(res)
        nxt = slstm_picard_next(int(inner.picard_iters or 0)) if ladder else None
        if ladder and nxt is not None and _picard_retry_needed(res, config):
            log.info("picard_adapt from_p=%d to_p=%d max_residual=%g",
                     int(inner.picard_iters or 0), nxt, res)
            inner = replace(inner, picard_iters=nxt)
            continue
        _fill_stats(cell, x, states, h0, replace(config, picard_iters=inner.picard_iters),
                    iters=int(config.max_iters), stats=stats, history=hist, known=res)
        return states


# ---------------------------------------------------------------------------
# Eq. 2.6 backward (newton/__init__.py:84-190, 765-918)
# ---------------------------------------------------------------------------

# Forward-thread hand-off for the duration of ``_NewtonFixedPoint.apply`` only;
# backward reads ``ctx`` alone.  Concurrent ``newton_apply`` calls with
# gradients are unsupported, as in the reference (newton/__init__.py:84-88).
_fwd_pack: dict[str, object] = {}


class _NewtonFixedPoint(torch.autograd.Function):
    """Implicit-function backward at the solved trajectory H* (eq. 2.6).

    Gradients never flow through the Newton iterations: backward solves the
    adjoint recursion ``mu_t = dL/dH_t + J_{t+1}^T mu_{t+1}`` at ``H*`` and
    contracts ``mu`` with the cell VJP (newton/__init__.py:91-190).
    """

    @staticmethod
    def forward(ctx, x_in: Tensor, h0_in: Tensor, *param_tensors: Tensor) -> Tensor:
        del param_tensors
        cell = _fwd_pack["cell"]
        config = _fwd_pack["config"]
        has_h0 = bool(_fwd_pack["has_h0"])
        h0_fwd = h0_in if has_h0 else None
        cs = _fwd_pack.get("cu_seqlens")
        ctx.cu_seqlens = cs
        ctx.cell = cell
        ctx.has_h0 = has_h0
        ctx.recompute = bool(config.recompute)
        ctx.fwd_config = config
        ctx.chunk_len = config.chunk_len
        with torch.no_grad():
            # Unchunked and not recomputing: keep W_x(x) for the backward's
            # cell VJP instead of projecting again.
            wx = None
            if config.chunk_len is None and not ctx.recompute:
                wx = cell.W_x(x_in)
            states = _newton_forward(cell, x_in, config, h0=h0_fwd, stats=_fwd_pack["stats"],
                                     wx=wx, cu_seqlens=cs)
        if ctx.recompute:
            ctx.save_for_backward(x_in, h0_in)
        elif wx is not None:
            ctx.save_for_backward(states, x_in, h0_in, wx)
        else:
            ctx.save_for_backward(states, x_in, h0_in)
        return states

    @staticmethod
    def backward(ctx, grad_states: Tensor):
        with _newton_precision_region(grad_states.device):
            return _NewtonFixedPoint._backward(ctx, grad_states)

    @staticmethod
    def _backward(ctx, grad_states: Tensor):
        if ctx.recompute:
            x_in, h0_in = ctx.saved_tensors
            h0_fwd = h0_in if ctx.has_h0 else None
            with torch.no_grad():
                states = _newton_forward(ctx.cell, x_in, ctx.fwd_config, h0=h0_fwd, stats=None,
                                         cu_seqlens=ctx.cu_seqlens)
        else:
            states, x_in, h0_in, *rest = ctx.saved_tensors
            wx = rest[0] if rest else None
            h0_fwd = h0_in if ctx.has_h0 else None
        if ctx.recompute:
            wx = None
        with torch.no_grad():
            if ctx.chunk_len is not None:
                grad_x, param_grads, grad_h0 = _eq26_vjp_chunked(
                    ctx.cell, states, x_in, grad_states, chunk_len=int(ctx.chunk_len), h0=h0_fwd
                )
            else:
                grad_x, param_grads, grad_h0 = _eq26_vjp(
                    ctx.cell, states, x_in, grad_states, h0=h0_fwd, wx=wx,
                    cu_seqlens=ctx.cu_seqlens
                )
        if not x_in.requires_grad:
            grad_x = None
        if not ctx.has_h0 or not h0_in.requires_grad:
            grad_h0 = None
        return (grad_x, grad_h0, *param_grads)


def _eq26_vjp(cell: nn.Module, states: Tensor, x: Tensor, partial: Tensor, *,
              h0: Tensor | None = None, wx: Tensor | None = None,
              cu_seqlens: Tensor | None = None):
    """``(grad_x, per-parameter grads, grad_h0)`` for diag ParaSLSTM and head ParaGRU.

    The reverse scan and the cell VJP run in one HIP op
    (``pararnn::slstm_backward_fused`` / ``pararnn::gru_head_backward_fused``);
    the clamp masks and the ``W_x`` VJP (two GEMMs and a column sum) follow the
    reference (solvers/vjp.py:103-120, 214-253, 288-306).
    """
    if wx is None:
        wx = cell.W_x(x)
    partial = partial.to(states.dtype)
    cap = cell.max_recurrent_norm
    if isinstance(cell, ParaSLSTM) and cell.mix == "diag":
        r_mix = cell.clipped_r()
        g_wx, g_r, g_h0, g_b = ops.slstm_backward_fused(wx, r_mix, h0, states, partial,
                                                       cu_seqlens, eps=cell.eps)
        determinism.maybe_check_fused_vjp_once(
            (g_r,),
            lambda: (ops.slstm_backward_fused(wx, r_mix, h0, states, partial, cu_seqlens,
                                              eps=cell.eps)[1],),
            cell_name=type(cell).__name__, shape=states.shape)
        g_r = g_r.to(cell.R.dtype)
        if cap is not None:
            g_r = g_r * (cell.R.abs() <= cap).to(g_r.dtype)
        by_name = {"R": g_r, "W_x.bias": g_b.reshape(-1).to(cell.W_x.bias.dtype)}
    elif isinstance(cell, ParaGRU) and cell.mix == "head":
        a_z, a_r, a_n = cell.clipped_a_head()
        g_wx, g_a, g_h0 = ops.gru_head_backward_fused(wx, a_z, a_r, a_n, h0, states, partial,
                                                      cu_seqlens)
        determinism.maybe_check_fused_vjp_once(
            (g_a,),
            lambda: (ops.gru_head_backward_fused(wx, a_z, a_r, a_n, h0, states, partial,
                                                 cu_seqlens)[1],),
            cell_name=type(cell).__name__, shape=states.shape)
        by_name = {}
        for i, name in enumerate(("A_z", "A_r", "A_n")):
            raw = getattr(cell, name)
            g = g_a[i].to(raw.dtype)
            if cap is not None:
                g = g * (raw.abs() <= cap).to(g.dtype)
            by_name[name] = g
    else:
        raise NotImplementedError(f"eq. 2.6 backward for {type(cell).__name__} is not built")
    gy = g_wx.reshape(-1, g_wx.shape[-1])
    xx = x.reshape(-1, x.shape[-1])
    grad_x = (gy @ cell.W_x.weight).reshape(x.shape)
    if "W_x.bias" not in by_name:
        by_name["W_x.bias"] = gy.sum(0)
    by_name["W_x.weight"] = _weight_grad(gy, xx)
    grads = tuple(
        by_name.get(n) if p.requires_grad else None for n, p in cell.named_parameters()
    )
    grad_h0 = None if h0 is None else g_h0.to(h0.dtype)
    return grad_x, grads, grad_h0


def _weight_grad(gy: Tensor, xx: Tensor) -> Tensor:
    """``gy^T xx`` over the B*T rows (the W_x gradient).  A single GEMM with a
    K = B*T reduction leaves too few output tiles to fill the GPU, so long
    reductions run as a batched GEMM over row blocks with fp32 partials, summed
    and rounded once."""
    n = int(gy.shape[0])
    if gy.is_cuda and n >= 65536 and gy.dtype in (torch.bfloat16, torch.float16, torch.float32):
        split = next((k for k in (16, 8, 4) if n % k == 0 and n // k >= 4096), 1)
        if split > 1:
            a = gy.view(split, n // split, -1).transpose(1, 2)
            b = xx.view(split, n // split, -1)
            if gy.dtype == torch.float32:
                return torch.bmm(a, b).sum(0)
            return torch.bmm(a, b, out_dtype=torch.float32).sum(0).to(gy.dtype)
    return gy.t() @ xx


def _eq26_vjp_chunked(cell: nn.Module, states: Tensor, x: Tensor, partial: Tensor, *,
                      chunk_len: int, h0: Tensor | None = None):
    """Eq. 2.6 on the windows of ``_newton_chunked``, last window first: the
    ``h0`` gradient of window i+1 adds to dL/dH at the last step of window i
    (newton/__init__.py:868-918)."""
    time = int(x.shape[1])
    acc_x = None
    acc = [None] * len(tuple(cell.parameters()))
    carry = None
    for t0 in reversed(range(0, time, int(chunk_len))):
        t1 = min(t0 + int(chunk_len), time)
        part = partial[:, t0:t1]
        if carry is not None:
            part = part.clone()
            part[:, -1] = part[:, -1] + carry
        h0_w = h0 if t0 == 0 else states[:, t0 - 1]
        gx, pg, gh0 = _eq26_vjp(cell, states[:, t0:t1], x[:, t0:t1], part, h0=h0_w)
        carry = gh0
        if acc_x is None:
            acc_x = x.new_zeros(x.shape)
        acc_x[:, t0:t1] = gx
        for i, g in enumerate(pg):
            if g is not None:
                acc[i] = g if acc[i] is None else acc[i] + g
    return acc_x, tuple(acc), (None if h0 is None else carry)
