"""``ParaRNN``: a stack of recurrent cells, each layer solved over the whole
sequence at once.

Public surface kept from the reference (``layers/para_rnn.py:27-288``): the
constructor and ``forward`` signatures and defaults, the attributes
(``layers``, ``config``, ``solver``, ``batch_first``, ``dropout``,
``output_hidden``, ``return_hidden``, ``hidden_layout``, ``last_stats``),
``reset_agreement_check`` / ``reset_parameters``, the exception types, and
the rule that ``solver='auto'`` means Newton in ``train()`` and the
sequential unroll in ``eval()``.

How it runs here: every layer is one call of a drop-in solver, either
``newton_apply`` (the fused HIP Newton solve; under autograd its eq. 2.6
backward) or ``sequential_apply`` (whose T=1 steps are the HIP decode
kernel), so the stack itself is host bookkeeping: checking shapes once,
threading each layer's readout into the next layer and collecting the
per-layer ``NewtonStats``.  ``hidden_layout='pytorch'`` concerns the
reference's ``ParaLSTM`` packing, a cell this build does not provide, so it
raises ``TypeError``.
"""

from __future__ import annotations

import inspect
import logging
import warnings
from collections.abc import Sequence
from dataclasses import dataclass
from typing import Literal

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from pararnn_amd.config import NewtonConfig, NewtonStats
from pararnn_amd.newton import newton_apply
from pararnn_amd.ragged import validate_cu_seqlens
from pararnn_amd.sequential import sequential_apply

log = logging.getLogger("pararnn_amd.layers")

SOLVERS = ("auto", "newton", "sequential")
HIDDEN_LAYOUTS = ("paper", "pytorch")

# Constructor knobs a deeper layer inherits from the template cell, when the
# template's class takes them and the template exposes them as attributes.
_SIZE_ARGS = {"self", "input_size", "hidden_size", "d_in", "d_h"}


@dataclass(frozen=True)
class CellShape:
    """What the stack needs to know about one cell (the reference's
    ``RNNCell`` protocol, cells/protocol.py:127-157): hidden width, number
    of state slots, which slot is the output, and the input width."""

    hidden: int
    slots: int
    out_slot: int | None
    features: int | None

    @classmethod
    def of(cls, cell: nn.Module) -> "CellShape":
        name = type(cell).__name__
        hidden = getattr(cell, "hidden_size", None)
        if hidden is None:
            hidden = getattr(cell, "d_h", None)
        if not isinstance(hidden, int) or hidden < 1:
            raise TypeError(f"{name}: hidden_size / d_h must be a positive int, got {hidden!r}")
        if not callable(getattr(cell, "step", None)):
            raise TypeError(f"{name}: a stacked cell needs a step(state_prev, x) method")
        slots = getattr(cell, "state_slots", 1)
        if slots not in (1, 2, 4):
            raise TypeError(f"{name}: state_slots must be 1, 2 or 4, got {slots!r}")
        features = getattr(cell, "input_size", None)
        if features is None:
            features = getattr(cell, "d_in", None)
        out_slot = None if slots == 1 else getattr(cell, "hidden_slot", 1)
        return cls(hidden, slots, out_slot, features if isinstance(features, int) else None)

    def state_shape(self, rows: int) -> tuple[int, ...]:
        return (rows, self.hidden) if self.slots == 1 else (rows, self.slots, self.hidden)

    def readout(self, states: Tensor) -> Tensor:
        """The part of ``(B, T, [slots,] d)`` states the next layer consumes."""
        return states if self.out_slot is None else states[:, :, self.out_slot, :]


def check_cell(cell: nn.Module) -> None:
    """Raise ``TypeError`` unless ``cell`` can be a layer of a ``ParaRNN``."""
    CellShape.of(cell)


def _placed(module: nn.Module, device, dtype) -> nn.Module:
    moves = {k: v for k, v in (("device", device), ("dtype", dtype)) if v is not None}
    return module.to(**moves) if moves else module


def _deeper_layer(template: nn.Module, device, dtype) -> nn.Module:
    """A fresh cell of the template's class reading the template's hidden
    width, with the template's other constructor knobs."""
    cls = type(template)
    params = inspect.signature(cls.__init__).parameters
    kw = {}
    for name, p in params.items():
        if name in _SIZE_ARGS or p.kind in (p.VAR_POSITIONAL, p.VAR_KEYWORD):
            continue
        if name in ("device", "dtype"):
            continue
        if hasattr(template, name):
            kw[name] = getattr(template, name)
    first = next(template.parameters(), None)
    if "device" in params:
        kw["device"] = device if device is not None else getattr(first, "device", None)
    if "dtype" in params:
        kw["dtype"] = dtype if dtype is not None else getattr(first, "dtype", None)
    width = CellShape.of(template).hidden
    try:
        cell = cls(input_size=width, hidden_size=width, **kw)
    except TypeError as exc:
        raise TypeError(
            f"cannot stack {cls.__name__} to num_layers > 1: its constructor must accept "
            f"input_size=hidden_size=<width> (or pass one cell per layer)"
        ) from exc
    return _placed(cell, device, dtype)


def _stack(cell, num_layers: int, device, dtype) -> list[nn.Module]:
    if isinstance(cell, (list, tuple)):
        if len(cell) == 0:
            raise ValueError("ParaRNN needs at least one cell")
        if num_layers not in (1, len(cell)):
            raise ValueError(
                f"num_layers={num_layers} but {len(cell)} cells were given; pass num_layers=1 "
                f"or num_layers=len(cells)"
            )
        for c in cell:
            check_cell(c)
        return [_placed(c, device, dtype) for c in cell]
    check_cell(cell)
    if num_layers < 1:
        raise ValueError(f"num_layers must be at least 1, got {num_layers}")
    first = _placed(cell, device, dtype)
    return [first] + [_deeper_layer(first, device, dtype) for _ in range(num_layers - 1)]


class ParaRNN(nn.Module):
    """Stacked RNN cells: Newton + scan in ``train()``, sequential ``step`` in ``eval()``.

    ``solver='auto'`` follows ``self.training``; ``'newton'`` / ``'sequential'``
    force one path.  Input ``(B, T, d_in)`` (``batch_first``) or
    ``(T, B, d_in)``; packed sequences as ``(1, N, d_in)`` with
    ``cu_seqlens``.  Multi-slot cells (sLSTM) emit their hidden slot unless
    ``output_hidden=False``; ``return_hidden=True`` also returns the final
    layer's last-step state.
    """

    def __init__(
        self,
        cell: nn.Module | Sequence[nn.Module],
        *,
        num_layers: int = 1,
        config: NewtonConfig | None = None,
        return_hidden: bool = False,
        output_hidden: bool | None = None,
        solver: Literal["auto", "newton", "sequential"] = "auto",
        batch_first: bool = True,
        hidden_layout: Literal["paper", "pytorch"] = "paper",
        dropout: float = 0.0,
        device: torch.device | str | None = None,
        dtype: torch.dtype | None = None,
    ) -> None:
        super().__init__()
        if solver not in SOLVERS:
            raise ValueError(f"unknown solver {solver!r}; choose from {SOLVERS}")
        if hidden_layout not in HIDDEN_LAYOUTS:
            raise ValueError(f"unknown hidden_layout {hidden_layout!r}; choose from "
                             f"{HIDDEN_LAYOUTS}")
        if not 0.0 <= dropout <= 1.0:
            raise ValueError(f"dropout is a probability in [0, 1], got {dropout}")
        self.layers = nn.ModuleList(_stack(cell, num_layers, device, dtype))
        if hidden_layout == "pytorch":
            raise TypeError(
                "hidden_layout='pytorch' is the ParaLSTM (h, c) packing; pararnn_amd stacks "
                "ParaSLSTM and ParaGRU, whose state layout is the paper's"
            )
        if dropout > 0 and len(self.layers) == 1:
            warnings.warn(
                f"dropout={dropout} acts between layers only, and this ParaRNN has a single "
                f"layer, so it has no effect",
                stacklevel=2,
            )
        self.config = config if config is not None else NewtonConfig()
        self.return_hidden = return_hidden
        self.solver = solver
        self.batch_first = batch_first
        self.hidden_layout = hidden_layout
        self.dropout = dropout
        self.last_stats: list[NewtonStats] = []
        self._agreement_verified = False
        top = CellShape.of(self.layers[-1])
        self.output_hidden = (top.out_slot is not None) if output_hidden is None else output_hidden

    # -- solver choice -------------------------------------------------------

    def _use_newton(self) -> bool:
        return {"newton": True, "sequential": False}.get(self.solver, self.training)

    def _effective_solver(self) -> str:
        return "newton" if self._use_newton() else "sequential"

    def reset_agreement_check(self) -> None:
        """Let ``config.verify_first_step`` run again on the next Newton forward."""
        self._agreement_verified = False

    def reset_parameters(self) -> None:
        for layer in self.layers:
            if callable(getattr(layer, "reset_parameters", None)):
                layer.reset_parameters()

    def extra_repr(self) -> str:
        return (f"solver={self.solver!r}, effective={self._effective_solver()}, "
                f"batch_first={self.batch_first}, dropout={self.dropout}, "
                f"output_hidden={self.output_hidden}, hidden_layout={self.hidden_layout!r}")

    # -- forward -------------------------------------------------------------

    def _initial_states(self, h0, rows: int, shapes: list[CellShape]) -> list[Tensor | None]:
        """One initial state (or None) per layer, shape-checked."""
        depth = len(shapes)
        if h0 is None:
            given: list = [None] * depth
        elif isinstance(h0, (list, tuple)):
            if len(h0) != depth:
                raise TypeError(f"h0 is a sequence of {len(h0)} states but the stack has "
                                f"{depth} layer(s); give one per layer (length {depth})")
            given = list(h0)
        elif depth == 1:
            given = [h0]
        else:
            raise TypeError(f"h0 for a {depth}-layer stack is a list/tuple of length {depth}")
        for i, (s, shape) in enumerate(zip(given, shapes)):
            want = shape.state_shape(rows)
            if s is not None and tuple(s.shape) != want:
                where = "h0" if depth == 1 else f"h0 for layer {i}"
                raise ValueError(f"{where} expected shape {want}, got {tuple(s.shape)}")
        return given

    def forward(
        self,
        x: Tensor,
        h0: Tensor | Sequence[Tensor] | None = None,
        cu_seqlens: Tensor | None = None,
    ) -> Tensor | tuple[Tensor, Tensor]:
        """``output`` (and, with ``return_hidden``, the final layer's last state)."""
        shapes = [CellShape.of(c) for c in self.layers]
        if x.ndim != 3:
            order = "(batch, time, features)" if self.batch_first else "(time, batch, features)"
            raise ValueError(f"expected a 3D input {order}, got shape {tuple(x.shape)}")
        want = shapes[0].features
        if want is not None and x.shape[-1] != want:
            raise ValueError(f"expected input features {want}, got {x.shape[-1]}")
        seq = x if self.batch_first else x.transpose(0, 1)
        rows = seq.shape[0]
        packed = None
        if cu_seqlens is not None:
            if rows != 1:
                raise ValueError(f"cu_seqlens needs x packed as batch 1, got batch {rows}")
            packed = validate_cu_seqlens(cu_seqlens, seq.shape[1])
            rows = int(packed.numel()) - 1
        starts = self._initial_states(h0, rows, shapes)

        newton = self._use_newton()
        if newton and packed is None:
            self._maybe_verify_first_step(x)
        stats: list[NewtonStats] = []
        self.last_stats = stats
        feats = seq
        last = len(self.layers) - 1
        for depth, (cell, shape, s0) in enumerate(zip(self.layers, shapes, starts)):
            if newton:
                st = NewtonStats()
                states = newton_apply(cell, feats, self.config, h0=s0, stats=st,
                                      cu_seqlens=packed)
                stats.append(st)
            else:
                states = sequential_apply(cell, feats, s0, cu_seqlens=packed)
            if depth < last:
                feats = shape.readout(states)
                if self.training and self.dropout > 0.0:
                    feats = F.dropout(feats, p=self.dropout, training=True)

        y = shapes[-1].readout(states) if self.output_hidden else states
        if not self.batch_first:
            y = y.transpose(0, 1)
        return (y, states[:, -1]) if self.return_hidden else y

    def _maybe_verify_first_step(self, x: Tensor) -> None:
        """``config.verify_first_step``: compare the two solvers once, on the
        first Newton forward, and raise ``AgreementError`` if they disagree."""
        if not self.config.verify_first_step or self._agreement_verified:
            return
        if torch.compiler.is_compiling():
            return
        # set first: the check itself runs this module's forward
        self._agreement_verified = True
        from pararnn_amd.verify import verify_agreement

        rep = verify_agreement(self, x, raise_on_fail=True)
        log.info("verify_first_step passed: max_abs=%g atol=%g", rep.max_abs, rep.atol)
