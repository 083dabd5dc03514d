"""``ParaRNN``: stacked cells, Newton + scan in ``train()``, sequential in ``eval()``
(reference ``layers/para_rnn.py:27-473``).

The wrapper is host logic over the drop-in entry points: each layer runs
``newton_apply`` (the fused HIP solve, with the eq. 2.6 backward under
autograd) or ``sequential_apply`` (whose T=1 case is the HIP decode step),
so a reference model switches by importing this class instead.  Same
constructor and ``forward`` signatures, defaults, validation, exception
types and ``last_stats``; the ``hidden_layout='pytorch'`` packing needs the
reference's ``ParaLSTM``, which this build does not provide (TypeError).
"""

from __future__ import annotations

import inspect
import logging
import warnings
from collections.abc import Sequence
from typing import Literal

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from pararnn_amd.config import NewtonConfig, NewtonStats
from pararnn_amd.newton import newton_apply
from pararnn_amd.ragged import validate_cu_seqlens
from pararnn_amd.sequential import sequential_apply

log = logging.getLogger("pararnn_amd.layers")

_SOLVERS = ("auto", "newton", "sequential")
_HIDDEN_LAYOUTS = ("paper", "pytorch")


def check_cell(cell: nn.Module) -> None:
    """The ``RNNCell`` surface a layer needs (reference cells/protocol.py:127-157)."""
    d_h = getattr(cell, "d_h", None)
    if d_h is None:
        d_h = getattr(cell, "hidden_size", None)
    if not isinstance(d_h, int) or d_h < 1:
        raise TypeError(
            f"{type(cell).__name__} needs integer d_h / hidden_size (hidden size), got {d_h!r}"
        )
    if not callable(getattr(cell, "step", None)):
        raise TypeError(f"{type(cell).__name__} needs a step(h_prev, x) method")
    slots = getattr(cell, "state_slots", 1)
    if slots not in (1, 2, 4):
        raise TypeError(f"{type(cell).__name__}.state_slots must be 1, 2, or 4, got {slots!r}")


class ParaRNN(nn.Module):
    """Stacked RNN cells: Newton + scan in ``train()``, sequential ``step`` in ``eval()``.

    ``solver='auto'`` follows ``self.training``; ``'newton'`` / ``'sequential'``
    force a path.  Input ``(B, T, d_in)`` (``batch_first``) or ``(T, B, d_in)``;
    packed sequences as ``(1, N, d_in)`` with ``cu_seqlens``.  Multi-slot cells
    (sLSTM) emit the hidden slot unless ``output_hidden=False``.
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
        if solver not in _SOLVERS:
            raise ValueError(f"solver must be one of {_SOLVERS}, got {solver!r}")
        if hidden_layout not in _HIDDEN_LAYOUTS:
            raise ValueError(
                f"hidden_layout must be one of {_HIDDEN_LAYOUTS}, got {hidden_layout!r}"
            )
        if not 0 <= dropout <= 1:
            raise ValueError(
                "dropout should be a number in range [0, 1] inclusive, but got a ratio of "
                f"{dropout}"
            )
        self.config = config or NewtonConfig()
        self.return_hidden = return_hidden
        self.solver = solver
        self.batch_first = batch_first
        self.hidden_layout = hidden_layout
        self.dropout = dropout
        self.last_stats: list[NewtonStats] = []
        self._agreement_verified = False
        self.layers = nn.ModuleList(_build_layers(cell, num_layers, device=device, dtype=dtype))
        if dropout > 0 and len(self.layers) == 1:
            warnings.warn(
                "dropout option adds dropout after all but last recurrent layer, so non-zero "
                f"dropout expects num_layers greater than 1, but got dropout={dropout} and "
                f"num_layers={len(self.layers)}",
                stacklevel=2,
            )
        if hidden_layout == "pytorch":
            raise TypeError(
                "hidden_layout='pytorch' is ParaLSTM only (nn.LSTM (h, c) vs paper (c, h)); "
                "pararnn_amd provides ParaSLSTM and ParaGRU"
            )
        if output_hidden is None:
            self.output_hidden = _hidden_slot(self.layers[-1]) is not None
        else:
            self.output_hidden = output_hidden

    def _use_newton(self) -> bool:
        if self.solver == "newton":
            return True
        if self.solver == "sequential":
            return False
        return self.training

    def _effective_solver(self) -> str:
        return "newton" if self._use_newton() else "sequential"

    def reset_agreement_check(self) -> None:
        """Allow ``verify_first_step`` to run again on the next Newton forward."""
        self._agreement_verified = False

    def reset_parameters(self) -> None:
        for cell in self.layers:
            reset = getattr(cell, "reset_parameters", None)
            if callable(reset):
                reset()

    def extra_repr(self) -> str:
        return (
            f"solver={self.solver!r}, effective={self._effective_solver()}, "
            f"batch_first={self.batch_first}, dropout={self.dropout}, "
            f"output_hidden={self.output_hidden}, hidden_layout={self.hidden_layout!r}"
        )

    def _maybe_verify_first_step(self, x: Tensor) -> None:
        """One parallel-vs-sequential check on the first Newton forward
        (``config.verify_first_step``)."""
        if not self.config.verify_first_step or self._agreement_verified:
            return
        if torch.compiler.is_compiling():
            return
        self._agreement_verified = True  # before verify re-enters forward
        from pararnn_amd.verify import verify_agreement

        report = verify_agreement(self, x, raise_on_fail=True)
        log.info("verify_first_step_ok max_abs=%g atol=%g", report.max_abs, report.atol)

    def forward(
        self,
        x: Tensor,
        h0: Tensor | Sequence[Tensor] | None = None,
        cu_seqlens: Tensor | None = None,
    ) -> Tensor | tuple[Tensor, Tensor]:
        """``output`` (and the final layer's last state with ``return_hidden``)."""
        _validate_input(x, self.layers[0], batch_first=self.batch_first)
        if not self.batch_first:
            x = x.transpose(0, 1)
        h0s = _split_h0(h0, len(self.layers))
        cs = None
        h0_batch = x.shape[0]
        if cu_seqlens is not None:
            if x.shape[0] != 1:
                raise ValueError(f"cu_seqlens packs x with batch=1, got batch={x.shape[0]}")
            cs = validate_cu_seqlens(cu_seqlens, x.shape[1])
            h0_batch = int(cs.numel()) - 1
        _validate_h0s(h0s, self.layers, batch=h0_batch)
        self.last_stats = []
        use_newton = self._use_newton()
        if use_newton and cs is None:
            self._maybe_verify_first_step(x)
        h = x
        n = len(self.layers)
        for i, cell in enumerate(self.layers):
            if use_newton:
                st = NewtonStats()
                h = newton_apply(cell, h, self.config, h0=h0s[i], stats=st, cu_seqlens=cs)
                self.last_stats.append(st)
            else:
                h = sequential_apply(cell, h, h0s[i], cu_seqlens=cs)
            if i + 1 < n:
                h = _next_layer_input(h, cell)
                if self.dropout > 0.0 and self.training:
                    h = F.dropout(h, p=self.dropout, training=True)
        last = h[:, -1]
        y = h
        slot = _hidden_slot(self.layers[-1])
        if self.output_hidden and slot is not None:
            y = h[:, :, slot, :]
        if not self.batch_first:
            y = y.transpose(0, 1)
        if self.return_hidden:
            return y, last
        return y


def _build_layers(cell, num_layers: int, *, device=None, dtype=None) -> list[nn.Module]:
    if isinstance(cell, (list, tuple)):
        if not cell:
            raise ValueError("cell list must be non-empty")
        if num_layers not in (1, len(cell)):
            raise ValueError(f"num_layers={num_layers} does not match len(cells)={len(cell)}")
        for c in cell:
            check_cell(c)
        return [_maybe_to(c, device, dtype) for c in cell]
    check_cell(cell)
    if num_layers < 1:
        raise ValueError(f"num_layers must be >= 1, got {num_layers}")
    layers = [_maybe_to(cell, device, dtype)]
    if num_layers > 1:
        layers += _extra_layers(layers[0], num_layers - 1, device=device, dtype=dtype)
    return layers


def _extra_layers(cell: nn.Module, n_extra: int, *, device=None, dtype=None) -> list[nn.Module]:
    """Deeper layers: the template's class with ``input_size = hidden_size``
    (layers/para_rnn.py:315-349)."""
    cls = type(cell)
    sig = inspect.signature(cls.__init__)
    kw = {n: getattr(cell, n) for n in ("max_recurrent_norm", "mix", "eps", "n_heads")
          if n in sig.parameters and hasattr(cell, n)}
    if device is None or dtype is None:
        p = next(cell.parameters(), None)
        device = device if device is not None else (p.device if p is not None else None)
        dtype = dtype if dtype is not None else (p.dtype if p is not None else None)
    if "device" in sig.parameters:
        kw["device"] = device
    if "dtype" in sig.parameters:
        kw["dtype"] = dtype
    hid = getattr(cell, "hidden_size", cell.d_h)
    out = []
    for _ in range(n_extra):
        try:
            extra = cls(input_size=hid, hidden_size=hid, **kw)
        except TypeError as exc:
            raise TypeError(
                f"{cls.__name__} cannot be stacked (num_layers>1): need "
                "type(cell)(input_size=hidden_size, hidden_size=hidden_size) or pass a list "
                "of cells"
            ) from exc
        out.append(_maybe_to(extra, device, dtype))
    return out


def _maybe_to(module: nn.Module, device, dtype) -> nn.Module:
    if device is None and dtype is None:
        return module
    kw = {}
    if device is not None:
        kw["device"] = device
    if dtype is not None:
        kw["dtype"] = dtype
    return module.to(**kw)


def _hidden_slot(cell: nn.Module) -> int | None:
    if getattr(cell, "state_slots", 1) == 1:
        return None
    return getattr(cell, "hidden_slot", 1)


def _next_layer_input(states: Tensor, cell: nn.Module) -> Tensor:
    slot = _hidden_slot(cell)
    return states if slot is None else states[:, :, slot, :]


def _input_size(cell: nn.Module) -> int | None:
    size = getattr(cell, "input_size", None)
    if size is None:
        size = getattr(cell, "d_in", None)
    return size if isinstance(size, int) else None


def _state_shape(cell: nn.Module, batch: int) -> tuple[int, ...]:
    hid = getattr(cell, "hidden_size", None) or cell.d_h
    slots = getattr(cell, "state_slots", 1)
    return (batch, hid) if slots == 1 else (batch, slots, hid)


def _validate_input(x: Tensor, cell: nn.Module, *, batch_first: bool) -> None:
    layout = "(batch, time, features)" if batch_first else "(time, batch, features)"
    if x.ndim != 3:
        raise ValueError(f"expected 3D input {layout}, got {x.ndim}D of shape {tuple(x.shape)}")
    d_in = _input_size(cell)
    if d_in is not None and x.shape[-1] != d_in:
        raise ValueError(
            f"expected input features {d_in}, got {x.shape[-1]} (shape {tuple(x.shape)})"
        )


def _validate_h0s(h0s, layers: nn.ModuleList, *, batch: int) -> None:
    for i, (h0, cell) in enumerate(zip(h0s, layers)):
        if h0 is None:
            continue
        expected = _state_shape(cell, batch)
        if tuple(h0.shape) != expected:
            where = f"h0 for layer {i}" if len(layers) > 1 else "h0"
            raise ValueError(f"{where} expected shape {expected}, got {tuple(h0.shape)}")


def _split_h0(h0, n_layers: int) -> list[Tensor | None]:
    if h0 is None:
        return [None] * n_layers
    if n_layers == 1:
        if isinstance(h0, (list, tuple)):
            if len(h0) != 1:
                raise TypeError(
                    f"h0 for 1 layer must be a state tensor or a length-1 sequence, got {len(h0)}"
                )
            return [h0[0]]
        return [h0]
    if not isinstance(h0, (list, tuple)) or len(h0) != n_layers:
        raise TypeError(f"h0 for {n_layers} layers must be a tuple/list of length {n_layers}")
    return list(h0)
