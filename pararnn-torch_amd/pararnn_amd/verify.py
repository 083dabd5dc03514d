"""Numerics contract: parallel Newton (HIP) vs the sequential unroll
(reference ``verify.py:28-217``)."""

from __future__ import annotations

import logging
from dataclasses import asdict, dataclass
from typing import Any

import torch
from torch import Tensor, nn

from pararnn_amd.config import NewtonConfig, NewtonStats
from pararnn_amd.layers import ParaRNN
from pararnn_amd.newton import newton_apply
from pararnn_amd.sequential import sequential_apply

log = logging.getLogger("pararnn_amd.verify")

_DEFAULT_ATOL_FP32 = 1e-4
_DEFAULT_ATOL_LOWP = 1e-2


@dataclass(frozen=True)
class AgreementReport:
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
    def __init__(self, message: str, report: AgreementReport) -> None:
        super().__init__(message)
        self.report = report


def default_agreement_atol(dtype: torch.dtype) -> float:
    """1e-4 for float32/float64, 1e-2 for float16/bfloat16."""
    return _DEFAULT_ATOL_LOWP if dtype in (torch.float16, torch.bfloat16) else _DEFAULT_ATOL_FP32


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
    """Compare the parallel Newton solve with the sequential unroll (``torch.allclose``
    rule) for a cell, a ``ParaRNN`` (both solvers on the same weights, in eval mode)
    or a block with ``.rnn: ParaRNN`` (verify.py:98-300)."""
    if x.dim() < 2:
        raise ValueError(f"x must be at least rank-2 (B, T, ...), got shape {tuple(x.shape)}")
    target = _resolve_target(module)
    atol_v = float(default_agreement_atol(x.dtype) if atol is None else atol)
    rtol_v = float(rtol)
    with torch.no_grad():
        if isinstance(target, ParaRNN):
            par, seq, stats = _compare_para_rnn(target, x)
            path = "para_rnn"
        else:
            cfg = config if config is not None else NewtonConfig()
            stats = NewtonStats()
            seq = sequential_apply(target, x, h0, cu_seqlens=cu_seqlens)
            par = newton_apply(target, x, cfg, h0=h0, stats=stats, cu_seqlens=cu_seqlens)
            path = "cell"
        diff = (par - seq).abs()
        max_abs = float(diff.amax().item())
        mean_abs = float(diff.float().mean().item())
        denom = seq.abs().clamp_min(torch.finfo(seq.dtype).eps)
        max_rel = float((diff / denom).amax().item())
        ok = bool(torch.allclose(par, seq, atol=atol_v, rtol=rtol_v))
    report = AgreementReport(
        ok=ok, max_abs=max_abs, max_rel=max_rel, mean_abs=mean_abs, atol=atol_v, rtol=rtol_v,
        shape=tuple(int(s) for s in par.shape), dtype=str(par.dtype).replace("torch.", ""),
        device=str(par.device), newton_iters=None if stats is None else int(stats.iters),
        max_residual=None if stats is None else float(stats.max_residual), path=path,
    )
    log.info("verify_agreement ok=%s max_abs=%g atol=%g", ok, max_abs, atol_v)
    if raise_on_fail and not ok:
        raise AgreementError(
            f"parallel vs sequential max_abs={max_abs:.3e} exceeds atol={atol_v:.3e} "
            f"(rtol={rtol_v:.3e}); shape={report.shape} dtype={report.dtype} path={path}",
            report,
        )
    return report


def _resolve_target(module: nn.Module) -> nn.Module:
    if isinstance(module, ParaRNN):
        return module
    rnn = getattr(module, "rnn", None)
    if isinstance(rnn, ParaRNN):
        return rnn
    if callable(getattr(module, "step", None)):
        return module
    raise TypeError(
        "verify_agreement expects an RNN cell with step(), a ParaRNN, or a block with "
        f".rnn: ParaRNN; got {type(module).__name__}"
    )


def _compare_para_rnn(model: ParaRNN, x: Tensor):
    """Both solvers on the same ``ParaRNN`` weights, in eval mode (no dropout)."""
    prev_solver, was_training = model.solver, model.training
    model.eval()
    try:
        model.solver = "sequential"
        seq = model(x)
        model.solver = "newton"
        par = model(x)
    finally:
        model.solver = prev_solver
        model.train(was_training)
    if isinstance(seq, tuple):
        seq = seq[0]
    if isinstance(par, tuple):
        par = par[0]
    return par, seq, (model.last_stats[-1] if model.last_stats else None)
