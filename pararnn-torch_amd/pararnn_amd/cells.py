"""The two cells of the hot path, with the reference's parameters and init.

``ParaSLSTM`` (``mix='diag'``) and ``ParaGRU`` (``mix='head'`` and ``'diag'``)
keep the reference's attribute names, parameter shapes, layouts and the
order of random draws in their constructors, so a ``state_dict`` of the
reference loads unchanged and ``torch.manual_seed(s)`` gives identical
weights (reference ``cells/para_slstm.py:80-200``, ``cells/para_gru.py:86-224``,
``weight_init.py:10-23``).

``step`` / ``step_with_jacobian`` are plain torch ops on any device: they
serve the sequential unroll, the post-solve residual gate and tests.  The
Newton solve itself runs the HIP kernels (``pararnn_amd.newton``).
"""

from __future__ import annotations

import math

import torch
from torch import Tensor, nn

SLSTM_CELL, SLSTM_NORMALIZER, SLSTM_STABILIZER, SLSTM_HIDDEN, SLSTM_SLOTS = 0, 1, 2, 3, 4

_DEFAULT_CAP = object()


def resolve_layer_sizes(input_size=None, hidden_size=None, *, d_in=None, d_h=None):
    """``input_size``/``hidden_size`` with aliases ``d_in``/``d_h`` (protocol.py:15-65)."""

    def pick(name, value, alias, alias_value):
        if value is not None and alias_value is not None and value != alias_value:
            raise ValueError(f"{name}={value!r} conflicts with {alias}={alias_value!r}")
        got = value if value is not None else alias_value
        if got is None:
            raise TypeError(f"missing {name} (or alias {alias})")
        if not isinstance(got, int):
            raise TypeError(f"{name} must be int, got {type(got).__name__}")
        return got

    a = pick("input_size", input_size, "d_in", d_in)
    b = pick("hidden_size", hidden_size, "d_h", d_h)
    if a < 1 or b < 1:
        raise ValueError(f"input_size and hidden_size must be positive, got {a}, {b}")
    return a, b


def xavier_gaussian_vec_(t: Tensor) -> None:
    """Normal(0, sqrt(1/numel)) — Xavier for a diagonal of size numel (weight_init.py:10-18)."""
    n = max(t.numel(), 1)
    nn.init.normal_(t, mean=0.0, std=math.sqrt(2.0 / (2 * n)))


def kaiming_uniform_linear_(w: Tensor) -> None:
    nn.init.kaiming_uniform_(w, a=math.sqrt(5))


class ParaSLSTM(nn.Module):
    """sLSTM cell with per-channel recurrent mix; state ``(..., 4, d_h)`` = (c, n, m, h).

    Only ``mix='diag'`` is provided by this build (the fused 4x4-block path).
    """

    def __init__(
        self,
        input_size: int | None = None,
        hidden_size: int | None = None,
        *,
        d_in: int | None = None,
        d_h: int | None = None,
        mix: str = "diag",
        n_heads: int | None = None,
        max_recurrent_norm: float | None = 0.5,
        eps: float = 1e-6,
        device=None,
        dtype=None,
    ) -> None:
        super().__init__()
        if mix not in ("diag", "dense", "head"):
            raise ValueError(f"mix must be one of ('diag', 'dense', 'head'), got {mix!r}")
        if mix != "diag":
            raise NotImplementedError(
                f"ParaSLSTM(mix={mix!r}) is not part of pararnn_amd; only mix='diag' is built"
            )
        if n_heads is not None:
            raise ValueError("n_heads is only for mix='head'")
        input_size, hidden_size = resolve_layer_sizes(input_size, hidden_size, d_in=d_in, d_h=d_h)
        fk = {"device": device, "dtype": dtype}
        self.input_size = self.d_in = input_size
        self.hidden_size = self.d_h = hidden_size
        self.state_slots = SLSTM_SLOTS
        self.hidden_slot = SLSTM_HIDDEN
        self.mix = mix
        self.jac_structure = "block4"
        self.max_recurrent_norm = max_recurrent_norm
        self.eps = eps
        self.n_heads = None
        self.d_head = None
        self.W_x = nn.Linear(input_size, 4 * hidden_size, bias=True, **fk)
        self.R = nn.Parameter(torch.empty(4, hidden_size, **fk))
        self.R_dense = None
        self.R_head = None
        self.reset_parameters()

    def extra_repr(self) -> str:
        return (f"{self.input_size}, {self.hidden_size}, mix={self.mix!r}, "
                f"max_recurrent_norm={self.max_recurrent_norm}, eps={self.eps}")

    def reset_parameters(self) -> None:
        kaiming_uniform_linear_(self.W_x.weight)
        nn.init.zeros_(self.W_x.bias)
        xavier_gaussian_vec_(self.R)

    def clipped_r(self) -> Tensor:
        cap = self.max_recurrent_norm
        return self.R if cap is None else self.R.clamp(-cap, cap)

    def _recurrent(self, h: Tensor) -> Tensor:
        return (self.clipped_r() * h.unsqueeze(-2)).reshape(*h.shape[:-1], 4 * self.d_h)

    def _acts(self, prev: Tensor, pre: Tensor) -> dict:
        c, n, m = prev[..., 0, :], prev[..., 1, :], prev[..., 2, :]
        zi, zf, zz, zo = pre.chunk(4, dim=-1)
        left = zf + m
        m_new = torch.maximum(left, zi)
        alpha = (left > zi).to(left.dtype) + 0.5 * (left == zi).to(left.dtype)
        i = torch.exp(zi - m_new)
        f = torch.exp(zf + m - m_new)
        z = torch.tanh(zz)
        n_new = f * n + i
        c_new = f * c + i * z
        o = torch.sigmoid(zo)
        denom = n_new + self.eps
        h_new = o * (c_new / denom)
        return dict(c=c, n=n, i=i, f=f, z=z, o=o, alpha=alpha, c_new=c_new, denom=denom,
                    new=torch.stack((c_new, n_new, m_new, h_new), dim=-2))

    def step(self, state_prev: Tensor, x: Tensor | None = None, *, wx: Tensor | None = None) -> Tensor:
        """One step ``f(state_prev, x)`` (para_slstm.py:216-239)."""
        if wx is None:
            wx = self.W_x(x)
        h = state_prev[..., SLSTM_HIDDEN, :]
        return self._acts(state_prev, wx + self._recurrent(h))["new"]

    def step_with_jacobian(self, state_prev: Tensor, x: Tensor | None = None, *,
                           wx: Tensor | None = None) -> tuple[Tensor, Tensor]:
        """Step and the per-channel ``(..., 4, 4, d_h)`` Jacobian ``[out, in, d]``
        (para_slstm.py:241-281, 378-446)."""
        if wx is None:
            wx = self.W_x(x)
        h = state_prev[..., SLSTM_HIDDEN, :]
        a = self._acts(state_prev, wx + self._recurrent(h))
        r = self.clipped_r()
        ri, rf, rz, ro = r[0], r[1], r[2], r[3]
        alpha = a["alpha"]
        beta = 1.0 - alpha
        i, f, z, o, c, n = a["i"], a["f"], a["z"], a["o"], a["c"], a["n"]
        dm_dh = alpha * rf + beta * ri
        di_dm = -i * alpha
        df_dm = f * beta
        di_dh = i * (ri - dm_dh)
        df_dh = f * (rf - dm_dh)
        dz_dh = (1.0 - z.square()) * rz
        do_dh = o * (1.0 - o) * ro
        zero = torch.zeros_like(f)
        cm = df_dm * c + di_dm * z
        ch = df_dh * c + di_dh * z + i * dz_dh
        nm = df_dm * n + di_dm
        nh = df_dh * n + di_dh
        inv = o / a["denom"]
        dn = -o * a["c_new"] / a["denom"].square()
        du = a["c_new"] / a["denom"]
        rows = (
            (f, zero, cm, ch),
            (zero, f, nm, nh),
            (zero, zero, alpha, dm_dh),
            (inv * f, dn * f, inv * cm + dn * nm, inv * ch + dn * nh + du * do_dh),
        )
        jac = torch.stack([torch.stack(row, dim=-2) for row in rows], dim=-3)
        return a["new"], jac


class ParaGRU(nn.Module):
    """Cho GRU with diagonal (``mix='diag'``) or block-diagonal per-head
    (``mix='head'``) recurrent weights; state ``(..., d_h)``.

    The fused path of this build is ``mix='head'``; the ``'diag'`` cell is
    provided for its ``step`` only.
    """

    def __init__(
        self,
        input_size: int | None = None,
        hidden_size: int | None = None,
        *,
        d_in: int | None = None,
        d_h: int | None = None,
        mix: str = "diag",
        n_heads: int | None = None,
        max_recurrent_norm=_DEFAULT_CAP,
        device=None,
        dtype=None,
    ) -> None:
        super().__init__()
        if mix not in ("diag", "head"):
            raise ValueError(f"mix must be one of ('diag', 'head'), got {mix!r}")
        input_size, hidden_size = resolve_layer_sizes(input_size, hidden_size, d_in=d_in, d_h=d_h)
        fk = {"device": device, "dtype": dtype}
        if max_recurrent_norm is _DEFAULT_CAP:
            max_recurrent_norm = None if mix == "head" else 0.5
        self.input_size = self.d_in = input_size
        self.hidden_size = self.d_h = hidden_size
        self.state_slots = 1
        self.mix = mix
        self.jac_structure = mix
        self.max_recurrent_norm = max_recurrent_norm
        self.n_heads = n_heads
        self.d_head = None
        self.a_z = self.a_r = self.a_n = None
        self.A_z = self.A_r = self.A_n = None
        self.W_x = nn.Linear(input_size, 3 * hidden_size, bias=True, **fk)
        if mix == "diag":
            if n_heads is not None:
                raise ValueError("n_heads is only for mix='head'")
            self.a_z = nn.Parameter(torch.empty(hidden_size, **fk))
            self.a_r = nn.Parameter(torch.empty(hidden_size, **fk))
            self.a_n = nn.Parameter(torch.empty(hidden_size, **fk))
        else:
            if n_heads is None or n_heads < 1 or hidden_size % n_heads != 0:
                raise ValueError(
                    f"mix='head' needs n_heads that divides hidden_size={hidden_size}, "
                    f"got {n_heads!r}"
                )
            self.d_head = hidden_size // n_heads
            shape = (n_heads, self.d_head, self.d_head)
            self.A_z = nn.Parameter(torch.empty(*shape, **fk))
            self.A_r = nn.Parameter(torch.empty(*shape, **fk))
            self.A_n = nn.Parameter(torch.empty(*shape, **fk))
            self.register_buffer("_eye_head", torch.eye(self.d_head, **fk), persistent=False)
        self.reset_parameters()

    def extra_repr(self) -> str:
        s = f"{self.input_size}, {self.hidden_size}, mix={self.mix!r}"
        if self.n_heads is not None:
            s += f", n_heads={self.n_heads}"
        return s + f", max_recurrent_norm={self.max_recurrent_norm}"

    def reset_parameters(self) -> None:
        kaiming_uniform_linear_(self.W_x.weight)
        nn.init.zeros_(self.W_x.bias)
        if self.a_z is not None:
            for v in (self.a_z, self.a_r, self.a_n):
                xavier_gaussian_vec_(v)
            return
        for A in (self.A_z, self.A_r, self.A_n):
            for hd in range(self.n_heads):
                w = torch.empty_like(A[hd], dtype=torch.float32)
                nn.init.orthogonal_(w, gain=0.25)
                A[hd].data.copy_(w.to(dtype=A.dtype))

    def clipped_a(self) -> tuple[Tensor, Tensor, Tensor]:
        if self.a_z is None:
            raise TypeError("clipped_a is for mix='diag'")
        cap = self.max_recurrent_norm
        if cap is None:
            return self.a_z, self.a_r, self.a_n
        return self.a_z.clamp(-cap, cap), self.a_r.clamp(-cap, cap), self.a_n.clamp(-cap, cap)

    def clipped_a_head(self) -> tuple[Tensor, Tensor, Tensor]:
        if self.A_z is None:
            raise TypeError("clipped_a_head is for mix='head'")
        cap = self.max_recurrent_norm
        if cap is None:
            return self.A_z, self.A_r, self.A_n
        return self.A_z.clamp(-cap, cap), self.A_r.clamp(-cap, cap), self.A_n.clamp(-cap, cap)

    def _acts(self, h: Tensor, wx: Tensor) -> dict:
        zx, rx, nx = wx.chunk(3, dim=-1)
        if self.mix == "diag":
            az, ar, an = self.clipped_a()
            z = torch.sigmoid(az * h + zx)
            r = torch.sigmoid(ar * h + rx)
            n = torch.tanh(an * (h * r) + nx)
            return dict(new=torch.lerp(h, n, z), h=h, z=z, r=r, n=n, a=(az, ar, an))
        az, ar, an = self.clipped_a_head()
        lead = h.shape[:-1]
        hv = h.reshape(*lead, self.n_heads, self.d_head)

        def mix(v, a):
            # h @ A per head (para_gru.py:414-416).  On the GPU as one GEMM
            # per head over every leading row: the broadcast
            # (..., 1, d) @ (H, d, d) form runs there as a batched GEMM of
            # single rows that re-reads A per row (12.7 ms instead of ~0.1 ms
            # at B=4, T=32768, H=8).  On the CPU the reference's own form, so
            # the eager step stays bit-identical to it.
            if v.is_cuda:
                rows = v.reshape(-1, self.n_heads, self.d_head).transpose(0, 1)
                return torch.bmm(rows, a.to(v.dtype)).transpose(0, 1).reshape(v.shape)
            return torch.matmul(v.unsqueeze(-2), a).squeeze(-2)

        zx, rx, nx = (t.reshape(*lead, self.n_heads, self.d_head) for t in (zx, rx, nx))
        z = torch.sigmoid(mix(hv, az) + zx)
        r = torch.sigmoid(mix(hv, ar) + rx)
        n = torch.tanh(mix(hv * r, an) + nx)
        new = torch.lerp(hv, n, z).reshape(*lead, self.d_h)
        return dict(new=new, h=hv, z=z, r=r, n=n, a=(az, ar, an))

    def step(self, h_prev: Tensor, x: Tensor | None = None, *, wx: Tensor | None = None) -> Tensor:
        """One GRU step (para_gru.py:283-313, 418-467)."""
        if wx is None:
            if x is None:
                raise ValueError("ParaGRU.step needs x or wx (precomputed W_x(x))")
            wx = self.W_x(x)
        return self._acts(h_prev, wx)["new"]

    def step_with_jacobian(self, h_prev: Tensor, x: Tensor | None = None, *,
                           wx: Tensor | None = None) -> tuple[Tensor, Tensor]:
        """Step and ``∂h'/∂h``: ``(..., d_h)`` diagonal or ``(..., H, d, d)`` ``[out, in]``
        per head (para_gru.py:344-412)."""
        if wx is None:
            if x is None:
                raise ValueError("ParaGRU.step needs x or wx (precomputed W_x(x))")
            wx = self.W_x(x)
        a = self._acts(h_prev, wx)
        z, r, n = a["z"], a["r"], a["n"]
        az, ar, an = a["a"]
        zp, rp, np_ = z * (1.0 - z), r * (1.0 - r), 1.0 - n.square()
        if self.mix == "diag":
            hh = a["h"]
            jac = (1.0 - z) + (n - hh) * zp * az + z * np_ * an * (r + hh * rp * ar)
            return a["new"], jac
        hv = a["h"]
        eye = self._eye_head.to(device=hv.device, dtype=hv.dtype)
        dz = zp.unsqueeze(-1) * az.transpose(-1, -2)
        dr = rp.unsqueeze(-1) * ar.transpose(-1, -2)
        du = torch.add(hv.unsqueeze(-1) * dr, r.unsqueeze(-1) * eye)
        dn = torch.matmul(np_.unsqueeze(-1) * an.transpose(-1, -2), du)
        jac = (1.0 - z).unsqueeze(-1) * eye + (n - hv).unsqueeze(-1) * dz + z.unsqueeze(-1) * dn
        return a["new"], jac
