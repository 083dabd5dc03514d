"""Parallel-vs-sequential agreement check.

Public surface kept from the reference (``verify.py:28-217``):
``verify_agreement``'s signature, the ``AgreementReport`` fields,
``AgreementError`` (a ``RuntimeError`` carrying the report),
``default_agreement_atol`` and its tolerances (1e-4 for fp32/fp64, 1e-2 for
fp16/bf16, ``rtol=0``), and the verdict rule, ``torch.allclose(parallel,
sequential, atol, rtol)``.

Here a check is a pair of runs of the same weights on the same input: the
parallel solve (``newton_apply``, the fused HIP Newton path) and the
sequential unroll (``sequential_apply``).  What the pair is depends on the
target: a cell runs both solvers directly; a ``ParaRNN`` (or a block holding
one as ``.rnn``) runs its own forward twice in ``eval()`` (no dropout) with
its ``solver`` switched, so the comparison covers the whole stack.
"""

from __future__ import annotations

import contextlib
import logging
from dataclasses import asdict, dataclass
from typing import Any, Callable

import torch
from torch import Tensor, nn

from pararnn_amd.config import NewtonConfig, NewtonStats
from pararnn_amd.layers import ParaRNN
from pararnn_amd.newton import newton_apply
from pararnn_amd.sequential import sequential_apply

log = logging.getLogger("pararnn_amd.verify")

ATOL_FULL_PRECISION = 1e-4
ATOL_HALF_PRECISION = 1e-2


@dataclass(frozen=True)
class AgreementReport:
    """Outcome of one ``verify_agreement`` call."""

    ok: bool
    max_abs: float
    max_rel: float
    mean_abs: float
    atol: float
    rtol: float
    shape: tuple[int, ...]
    dtype: str
    device: str
    newton_iters: int | None = None
    max_residual: float | None = None
    path: str = "cell"

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)


class AgreementError(RuntimeError):
    """Raised by ``verify_agreement(..., raise_on_fail=True)``; ``.report`` holds the numbers."""

    def __init__(self, message: str, report: AgreementReport) -> None:
        super().__init__(message)
        self.report = report


def default_agreement_atol(dtype: torch.dtype) -> float:
    """1e-2 for float16 / bfloat16, else 1e-4."""
    half = dtype in (torch.float16, torch.bfloat16)
    return ATOL_HALF_PRECISION if half else ATOL_FULL_PRECISION


# A pair runner returns (parallel output, sequential output, stats of the
# last Newton solve or None).
_Pair = tuple[Tensor, Tensor, "NewtonStats | None"]


@contextlib.contextmanager
def _forced_solver(model: ParaRNN, solver: str):
    """``model`` in eval mode with ``solver`` forced; both restored after."""
    saved = (model.solver, model.training)
    model.eval()
    model.solver = solver
    try:
        yield model
    finally:
        model.solver = saved[0]
        model.train(saved[1])


def _first(out):
    return out[0] if isinstance(out, tuple) else out


def _stack_pair(model: ParaRNN) -> Callable[..., _Pair]:
    def run(x, config, h0, cu_seqlens) -> _Pair:
        with _forced_solver(model, "sequential"):
            seq = _first(model(x))
        with _forced_solver(model, "newton"):
            par = _first(model(x))
            stats = model.last_stats[-1] if model.last_stats else None
        return par, seq, stats

    return run


def _cell_pair(cell: nn.Module) -> Callable[..., _Pair]:
    def run(x, config, h0, cu_seqlens) -> _Pair:
        stats = NewtonStats()
        seq = sequential_apply(cell, x, h0, cu_seqlens=cu_seqlens)
        par = newton_apply(cell, x, config if config is not None else NewtonConfig(),
                           h0=h0, stats=stats, cu_seqlens=cu_seqlens)
        return par, seq, stats

    return run


def _pair_for(module: nn.Module) -> tuple[Callable[..., _Pair], str]:
    for candidate in (module, getattr(module, "rnn", None)):
        if isinstance(candidate, ParaRNN):
            return _stack_pair(candidate), "para_rnn"
    if callable(getattr(module, "step", None)):
        return _cell_pair(module), "cell"
    raise TypeError(
        f"verify_agreement needs a cell with step(), a ParaRNN or a module whose .rnn is a "
        f"ParaRNN; got {type(module).__name__}"
    )


def verify_agreement(
    module: nn.Module,
    x: Tensor,
    *,
    config: NewtonConfig | None = None,
    h0: Tensor | None = None,
    atol: float | None = None,
    rtol: float = 0.0,
    raise_on_fail: bool = False,
    cu_seqlens: Tensor | None = None,
) -> AgreementReport:
    """Run the parallel Newton solve and the sequential unroll of ``module`` on
    ``x`` and report how far apart they are.  ``ok`` is ``torch.allclose``
    with ``atol`` (default by dtype, ``default_agreement_atol``) and ``rtol``.
    ``config``, ``h0`` and ``cu_seqlens`` apply to a bare cell; a ``ParaRNN``
    uses its own."""
    if x.dim() < 2:
        raise ValueError(f"x must have at least 2 dims (batch, time, ...), got {tuple(x.shape)}")
    run, path = _pair_for(module)
    tol_a = float(atol) if atol is not None else default_agreement_atol(x.dtype)
    tol_r = float(rtol)
    with torch.no_grad():
        par, seq, stats = run(x, config, h0, cu_seqlens)
        gap = (par - seq).abs()
        floor = torch.finfo(seq.dtype).eps
        report = AgreementReport(
            ok=bool(torch.allclose(par, seq, atol=tol_a, rtol=tol_r)),
            max_abs=float(gap.max()),
            max_rel=float((gap / seq.abs().clamp_min(floor)).max()),
            mean_abs=float(gap.float().mean()),
            atol=tol_a,
            rtol=tol_r,
            shape=tuple(par.shape),
            dtype=str(par.dtype).removeprefix("torch."),
            device=str(par.device),
            newton_iters=None if stats is None else int(stats.iters),
            max_residual=None if stats is None else float(stats.max_residual),
            path=path,
        )
    log.info("verify_agreement path=%s ok=%s max_abs=%g atol=%g", path, report.ok,
             report.max_abs, tol_a)
    if raise_on_fail and not report.ok:
        raise AgreementError(
            f"parallel and sequential solves differ by up to {report.max_abs:.3e} (atol "
            f"{tol_a:.3e}, rtol {tol_r:.3e}) on {report.shape} {report.dtype} ({path})",
            report,
        )
    return report
