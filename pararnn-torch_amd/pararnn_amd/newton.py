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
* after the solve the residual gate re-evaluates ``max |F|`` with the cell's
  torch ``step`` and raises :class:`NewtonDivergenceError` above
  ``residual_fail``.

The Newton solve itself never runs on the CPU: inputs on another device, or
backends this build does not provide ('eager', 'triton',
'context_parallel'), raise instead of falling back.
"""

from __future__ import annotations

import logging
import math
from dataclasses import replace

import torch
from torch import Tensor, nn

from pararnn_amd import ops
from pararnn_amd.cells import SLSTM_HIDDEN, ParaGRU, ParaSLSTM
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
    if x.device.type != "cuda" or x.dtype not in (torch.float32, torch.bfloat16):
        return False
    if isinstance(cell, ParaSLSTM):
        return cell.mix == "diag"
    if isinstance(cell, ParaGRU):
        return cell.mix == "head" and cell.d_head == 64
    return False


def _fused_error(cell: nn.Module, x: Tensor) -> str:
    return (
        "scan_backend='fused' in pararnn_amd needs ParaSLSTM(mix='diag') or "
        "ParaGRU(mix='head', d_head=64) on a ROCm GPU in float32/bfloat16 "
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
    if requested in ("eager", "triton", "context_parallel"):
        raise NotImplementedError(
            f"scan_backend={requested!r} is not provided by pararnn_amd; its Newton solve "
            "runs the fused HIP kernels ('fused' / 'auto')"
        )
    if not _fusable(cell, x):
        raise TypeError(_fused_error(cell, x))
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
            raise TypeError("block_table fused Newton is mix='diag' ParaGRU only")
        a_z, a_r, a_n = cell.clipped_a_head()
        return ops.newton_gru_head_fused(
            wx, a_z, a_r, a_n, h0, cu_seqlens, max_iters=max_iters, omega=omega
        )
    if isinstance(cell, ParaSLSTM) and cell.mix == "diag":
        if cu_seqlens is not None:
            raise TypeError("pararnn_amd fused ParaSLSTM does not take cu_seqlens")
        r = cell.clipped_r()
        states = ops.slstm_init_fused(wx, r, h0, picard_iters=int(picard_iters), eps=cell.eps)
        return ops.newton_slstm_fused(
            wx, r, h0, states, block_table,
            max_iters=max_iters, omega=omega, eps=cell.eps, log_coords=log_coords,
            scan_tile=scan_tile, time_loop=fused_time_loop,
            window_len=0 if fused_window_len is None else int(fused_window_len),
        )
    raise TypeError(_fused_error(cell, wx))


def _fill_stats(cell, x, states, h0, config, *, iters, stats, history=(), known=None) -> None:
    """Residual gate (newton/__init__.py:582-636): one extra cell step over T."""
    if stats is None and config.residual_fail is None:
        return
    if known is None:
        pred = cell.step(_prepend(states, h0), x)
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


def _newton_solve(cell, x, config, *, h0, stats) -> Tensor:
    if config.chunk_len is not None:
        return _newton_chunked(cell, x, config, h0=h0, stats=stats)
    if config.fused_early_exit:
        raise TypeError("fused_early_exit is not provided by pararnn_amd")
    wx = cell.W_x(x)
    states = fused_newton(
        cell, wx,
        max_iters=int(config.max_iters), omega=float(config.omega), h0=h0,
        log_coords=config.coords == "log", picard_iters=int(config.picard_iters or 0),
        scan_tile=config.scan_tile, fused_time_loop=config.fused_time_loop,
        fused_window_len=config.fused_window_len,
    )
    if not torch.compiler.is_compiling():
        _fill_stats(cell, x, states, h0, config, iters=int(config.max_iters), stats=stats)
    return states


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


def _newton_forward(cell, x, config, *, h0, stats) -> Tensor:
    if config.chunk_len is not None:
        return _newton_chunked(cell, x, config, h0=h0, stats=stats)
    if not (config.picard_adapt and isinstance(cell, ParaSLSTM)) or torch.compiler.is_compiling():
        return _newton_solve(cell, x, config, h0=h0, stats=stats)
    # Adaptive Picard ladder (picard.py:105-158).
    cfg = config
    while True:
        st = stats if stats is not None else NewtonStats()
        states = _newton_solve(cell, x, replace(cfg, residual_fail=None), h0=h0, stats=st)
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
                        history=st.residual_history, known=res)
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
    config = _resolve_backend(cell, x, config)
    if cu_seqlens is not None:
        raise TypeError(
            "packed cu_seqlens batches are not provided by pararnn_amd; pad to a rectangular batch"
        )
    if block_table is not None:
        if config.chunk_len is not None:
            raise ValueError("block_table cannot be combined with chunk_len")
        raise TypeError("block_table (paged h0) is not provided by pararnn_amd")
    params = tuple(cell.parameters())
    needs_grad = torch.is_grad_enabled() and (
        x.requires_grad
        or (h0 is not None and h0.requires_grad)
        or any(p.requires_grad for p in params)
    )
    if needs_grad:
        raise NotImplementedError(
            "pararnn_amd provides the Newton forward only; the eq. 2.6 backward is not built "
            "yet. Run newton_apply under torch.no_grad() / torch.inference_mode()."
        )
    return _newton_forward(cell, x, config, h0=h0, stats=stats)
