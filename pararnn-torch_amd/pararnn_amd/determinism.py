"""Run-to-run determinism under ``torch.use_deterministic_algorithms(True)``.

Mirrors pararnn/determinism.py:41-113 of the reference: when torch's
deterministic flag is on, the first fused eq. 2.6 VJP is run a second time on
the same inputs and a single warning is logged if the recurrent parameter
gradients differ bit for bit.

On this path the flag also switches the HIP library's look-back scans into
their deterministic mode (``prnn_set_deterministic``, set before each sLSTM
launch): every tile's carry is then the serial chain of published tile
aggregates, so forward states, ``grad_x``/``grad_h0`` and the parameter
gradients are bit-identical between runs.  The head GRU scans are
deterministic in either mode, and every reduction (R, A, bias, the split-K
``W_x`` partials) sums in a fixed order with no atomics.  The reference's
``CUBLAS_WORKSPACE_CONFIG`` advice (determinism.py:48-61) concerns cuBLAS
workspaces and has no counterpart on ROCm's GEMM path.
"""

from __future__ import annotations

import logging
from typing import Callable, Sequence

import torch
from torch import Tensor

log = logging.getLogger("pararnn_amd")

_CHECKED_VJP = False
_WARNED_VJP = False


def deterministic_algorithms_enabled() -> bool:
    """``torch.are_deterministic_algorithms_enabled()`` (determinism.py:41-45)."""
    fn = getattr(torch, "are_deterministic_algorithms_enabled", None)
    return bool(fn()) if fn is not None else False


def param_grads_bitmatch(a: Sequence[Tensor | None], b: Sequence[Tensor | None]) -> bool:
    """True when both sequences hold the same tensors bit for bit (None where
    the other is None) -- determinism.py:63-74."""
    if len(a) != len(b):
        return False
    for x, y in zip(a, b):
        if x is None or y is None:
            if x is not y:
                return False
            continue
        if x.shape != y.shape or x.dtype != y.dtype:
            return False
        # Byte view: NaN payloads compare equal to themselves, -0 differs from +0.
        if not torch.equal(x.contiguous().view(torch.uint8), y.contiguous().view(torch.uint8)):
            return False
    return True


def maybe_check_fused_vjp_once(first: Sequence[Tensor | None],
                               rerun: Callable[[], Sequence[Tensor | None]],
                               *, cell_name: str, shape: tuple) -> None:
    """On the first fused VJP under deterministic algorithms, run it again
    (``rerun``) and warn once if the recurrent parameter gradients drift
    (determinism.py:77-113).  Does nothing when the flag is off."""
    global _CHECKED_VJP, _WARNED_VJP
    if _CHECKED_VJP or not deterministic_algorithms_enabled():
        return
    _CHECKED_VJP = True
    second = rerun()
    if param_grads_bitmatch(first, second) or _WARNED_VJP:
        return
    _WARNED_VJP = True
    log.warning(
        "ParaRNN fused eq. 2.6 VJP parameter gradients differed across two identical calls "
        "while torch.use_deterministic_algorithms(True); expected bit-stable scans and "
        "fixed-order reductions. cell=%s states=%s", cell_name, tuple(shape),
    )


def reset_checks() -> None:
    """Forget that the one-shot check ran (for tests)."""
    global _CHECKED_VJP, _WARNED_VJP
    _CHECKED_VJP = False
    _WARNED_VJP = False
