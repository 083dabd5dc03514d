"""Solver knobs, statistics and the divergence error.

Same fields, defaults and validation as the reference's ``NewtonConfig`` /
``NewtonStats`` / ``NewtonDivergenceError``
(``solvers/newton/config.py:10-267``), so configs written for the reference
construct unchanged.  Knobs that select paths this build does not provide
(log coordinates, windowed fused walk, Thomas tiles, context parallelism)
validate as in the reference and are rejected with ``TypeError`` at dispatch.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass

# Library constants (config.py:10-28).
_DEFAULT_RESIDUAL_ATOL = 1e-5
LIBRARY_NEWTON_ITERS = 3
_DEFAULT_RESIDUAL_FAIL = 1.0
_RESIDUAL_WARN = 1e-3
FUSED_WINDOW_LENS = (32, 64, 128)
FUSED_WINDOW_DEFAULT = 64


class NewtonDivergenceError(RuntimeError):
    """``max |F|`` after the K Newton steps exceeds ``NewtonConfig.residual_fail``."""


@dataclass
class NewtonStats:
    """Filled in place by ``newton_apply(..., stats=...)`` (config.py:31-56)."""

    max_residual: float = float("nan")
    iters: int = 0
    scan_backend: str = ""
    picard_iters: int = 0
    residual_history: tuple[float, ...] = ()


@dataclass
class NewtonConfig:
    """Parallel Newton + scan knobs (config.py:59-187)."""

    max_iters: int | None = LIBRARY_NEWTON_ITERS
    omega: float = 1.0
    scan_backend: str = "auto"
    jacobian: str = "auto"
    jac_structure: str | None = None
    residual_atol: float | None = _DEFAULT_RESIDUAL_ATOL
    residual_fail: float | None = _DEFAULT_RESIDUAL_FAIL
    coords: str = "native"
    chunk_len: int | None = None
    picard_iters: int | None = None
    picard_adapt: bool | None = None
    picard_retry_atol: float | None = _RESIDUAL_WARN
    newton_iters_by_t: Mapping[int, int] | None = None
    scan_tile: str = "assoc"
    fused_time_loop: bool = False
    fused_window_len: int | None = None
    recompute: bool = False
    fused_early_exit: bool = False
    verify_first_step: bool = False
    newton_backtrack: bool = False


def compile_safe_config(*, scan_backend: str = "eager") -> NewtonConfig:
    """Fixed-K preset without host syncs (config.py:196-221)."""
    return NewtonConfig(
        max_iters=LIBRARY_NEWTON_ITERS,
        scan_backend=scan_backend,
        residual_atol=None,
        residual_fail=None,
        picard_adapt=False,
    )


def validate_config(config: NewtonConfig) -> None:
    """Reject malformed knob values with ``ValueError`` (config.py:224-267)."""
    c = config
    if c.scan_backend not in ("auto", "eager", "triton", "fused", "context_parallel"):
        raise ValueError(f"unknown scan backend {c.scan_backend!r}")
    if c.jacobian not in ("auto", "analytic", "autograd"):
        raise ValueError(f"unknown jacobian {c.jacobian!r}")
    if c.coords not in ("native", "log"):
        raise ValueError(f"unknown newton coords {c.coords!r}")
    if c.chunk_len is not None and int(c.chunk_len) < 1:
        raise ValueError(f"chunk_len must be >= 1, got {c.chunk_len!r}")
    if c.max_iters is not None and int(c.max_iters) < 0:
        raise ValueError(f"max_iters must be >= 0 or None, got {c.max_iters!r}")
    if c.picard_iters is not None and int(c.picard_iters) < 0:
        raise ValueError(f"picard_iters must be >= 0, got {c.picard_iters!r}")
    if c.picard_retry_atol is not None and float(c.picard_retry_atol) < 0:
        raise ValueError(f"picard_retry_atol must be >= 0 or None, got {c.picard_retry_atol!r}")
    if c.residual_fail is not None and float(c.residual_fail) < 0:
        raise ValueError(f"residual_fail must be >= 0 or None, got {c.residual_fail!r}")
    if c.newton_iters_by_t is not None:
        if c.max_iters is not None:
            raise ValueError("newton_iters_by_t requires max_iters=None (auto K*(T))")
        if not c.newton_iters_by_t:
            raise ValueError("newton_iters_by_t must be a non-empty mapping")
        for k, v in c.newton_iters_by_t.items():
            if int(k) < 1 or int(v) < 0:
                raise ValueError(f"newton_iters_by_t bad entry T={k!r} -> K={v!r}")
    if c.scan_tile not in ("assoc", "seq", "thomas", "thomas2", "thomas4"):
        raise ValueError(f"unknown scan_tile {c.scan_tile!r}")
    if c.fused_time_loop and c.chunk_len is not None:
        raise ValueError("fused_time_loop and chunk_len both set; pick one windowed path")
    if c.fused_time_loop and c.coords == "log":
        raise ValueError("fused_time_loop is native coords only")
    if c.fused_window_len is not None:
        w = int(c.fused_window_len)
        if w not in FUSED_WINDOW_LENS:
            raise ValueError(f"fused_window_len must be one of {FUSED_WINDOW_LENS}, got {w}")
        if not c.fused_time_loop:
            raise ValueError("fused_window_len requires fused_time_loop=True")
    if c.fused_early_exit:
        if c.residual_atol is None:
            raise ValueError("fused_early_exit requires residual_atol (got None)")
        if c.fused_time_loop:
            raise ValueError("fused_early_exit cannot combine with fused_time_loop")


def lookup_iters_by_t(schedule: Mapping[int, int], seq_len: int) -> int:
    """Largest key ``<= seq_len`` wins, else the smallest key (k_star.py:31-42)."""
    if not schedule:
        raise ValueError("empty newton_iters_by_t schedule")
    keys = sorted(int(k) for k in schedule)
    chosen = int(schedule[keys[0]])
    for k in keys:
        if k > seq_len:
            break
        chosen = int(schedule[k])
    return chosen
