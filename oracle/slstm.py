"""ParaSLSTM ``mix='diag'`` eager restatement (test infrastructure only).

Restates, on the CPU:
* the cell ``f`` — reference ``cells/para_slstm.py:202-207`` (clamp of R),
  ``:304-311`` (recurrent mix ``R * h``), ``:347-376`` (``_acts_from_pre``);
* the 4x4 per-channel Jacobian — ``cells/para_slstm.py:378-446, 530-534``;
* the frozen-gate scan and Picard warm start — ``solvers/slstm_picard.py:51-107,
  143-181`` and the auto depth ``solvers/newton/picard.py:22-45``;
* the eager Newton loop — ``solvers/newton/__init__.py:467-549`` with
  ``layout.py:78-90`` (``prepend_state``);
* the sequential unroll — ``solvers/sequential.py:22-86``.

State layout ``(B, T, 4, d)`` with slots ``(c, n, m, h)``; ``wx`` is
``(B, T, 4d)`` with gate blocks ``(i, f, z, o)``.  Every expression keeps the
reference's operand order, since bf16 tensors round after each op.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor

from oracle.scan import scan_block4, scan_diag

C, N, M, H = 0, 1, 2, 3


@dataclass
class SLSTMParams:
    W: Tensor  # (4d, d_in)
    b: Tensor  # (4d,)
    R: Tensor  # (4, d) raw parameter (clamped on use)
    eps: float = 1e-6
    cap: float | None = 0.5

    @property
    def d(self) -> int:
        return self.R.shape[-1]

    def r(self) -> Tensor:
        # para_slstm.py:202-207
        return self.R if self.cap is None else self.R.clamp(-self.cap, self.cap)

    def wx(self, x: Tensor) -> Tensor:
        return F.linear(x, self.W, self.b)


def auto_picard(seq_len: int) -> int:
    """Auto Picard depth by T (picard.py:22-45): 1 / 3 / 5."""
    return 1 if seq_len <= 64 else (3 if seq_len <= 2048 else 5)


def _pre(p: SLSTMParams, wx: Tensor, h: Tensor) -> Tensor:
    # para_slstm.py:304-311 then ``wx + _recurrent(h)`` at :237, :273
    rec = (p.r() * h.unsqueeze(-2)).reshape(*h.shape[:-1], 4 * p.d)
    return wx + rec


def _acts(p: SLSTMParams, prev: Tensor, pre: Tensor) -> dict:
    # para_slstm.py:347-376
    c, n, m = prev[..., C, :], prev[..., N, :], prev[..., M, :]
    zi, zf, zz, zo = pre.chunk(4, dim=-1)
    left = zf + m
    m_new = torch.maximum(left, zi)
    # torch.maximum subgradient: 1 / 0.5 / 0 (para_slstm.py:530-534)
    alpha = (left > zi).to(left.dtype) + 0.5 * (left == zi).to(left.dtype)
    i = torch.exp(zi - m_new)
    f = torch.exp(zf + m - m_new)
    z = torch.tanh(zz)
    n_new = f * n + i
    c_new = f * c + i * z
    o = torch.sigmoid(zo)
    denom = n_new + p.eps
    h_new = o * (c_new / denom)
    return dict(c=c, n=n, m=m, i=i, f=f, z=z, o=o, alpha=alpha, c_new=c_new,
                n_new=n_new, denom=denom,
                new=torch.stack((c_new, n_new, m_new, h_new), dim=-2))


def slstm_step(p: SLSTMParams, prev: Tensor, wx: Tensor) -> Tensor:
    """One step ``f(prev, x)`` from the pre-projected gates."""
    return _acts(p, prev, _pre(p, wx, prev[..., H, :]))["new"]


def _jac_rows(a: dict, r: Tensor) -> list[list[Tensor]]:
    # para_slstm.py:391-446, rows = out slot, columns = in slot
    r_i, r_f, r_z, r_o = r[0], r[1], r[2], r[3]
    alpha = a["alpha"]
    beta = 1.0 - alpha
    i, f, z, o, c, n = a["i"], a["f"], a["z"], a["o"], a["c"], a["n"]
    dm_dh = alpha * r_f + beta * r_i
    di_dm = -i * alpha
    df_dm = f * beta
    di_dh = i * (r_i - dm_dh)
    df_dh = f * (r_f - dm_dh)
    dz_dh = (1.0 - z.square()) * r_z
    do_dh = o * (1.0 - o) * r_o
    zero = torch.zeros_like(f)
    cm = df_dm * c + di_dm * z
    ch = df_dh * c + di_dh * z + i * dz_dh
    nm = df_dm * n + di_dm
    nh = df_dh * n + di_dh
    inv = o / a["denom"]
    dn = -o * a["c_new"] / a["denom"].square()
    du = a["c_new"] / a["denom"]
    hc = inv * f
    hn = dn * f
    hm = inv * cm + dn * nm
    hh = inv * ch + dn * nh + du * do_dh
    return [
        [f, zero, cm, ch],
        [zero, f, nm, nh],
        [zero, zero, alpha, dm_dh],
        [hc, hn, hm, hh],
    ]


def slstm_jacobian(p: SLSTMParams, prev: Tensor, wx: Tensor) -> tuple[Tensor, Tensor]:
    """``(f(prev), J)`` with J ``(..., 4, 4, d)`` laid out ``[out, in, d]``."""
    a = _acts(p, prev, _pre(p, wx, prev[..., H, :]))
    rows = _jac_rows(a, p.r())
    jac = torch.stack([torch.stack(row, dim=-2) for row in rows], dim=-3)
    return a["new"], jac


def prepend(states: Tensor, h0: Tensor | None) -> Tensor:
    """Previous state at each t: ``h0`` (or zeros) then ``states[:, :-1]`` (layout.py:78-90)."""
    out = states.new_empty(states.shape)
    out[:, 0] = 0 if h0 is None else h0
    out[:, 1:] = states[:, :-1]
    return out


def frozen_gate_scan(pre: Tensor, eps: float, h0: Tensor | None = None) -> Tensor:
    """sLSTM trajectory with gates frozen in ``pre`` (slstm_picard.py:51-107).

    fp32 algebra: the stabiliser is ``m_t = p_t + max(cummax(z_i - p)_t, m0)``
    with ``p = cumsum(z_f)``; ``n`` and ``c`` are diagonal scans sharing the
    forget factor; ``h`` is the readout.  Output in ``pre``'s dtype.
    """
    bsz = pre.shape[0]
    d = pre.shape[-1] // 4
    out_dtype = pre.dtype
    q = pre.float()
    zi, zf, zz, zo = q.chunk(4, dim=-1)
    if h0 is None:
        c0 = n0 = m0 = q.new_zeros(bsz, d)
    else:
        g = h0.float()
        c0, n0, m0 = g[:, C], g[:, N], g[:, M]
    p = zf.cumsum(dim=1)
    m = p + torch.maximum((zi - p).cummax(dim=1).values, m0.unsqueeze(1))
    m_prev = torch.cat((m0.unsqueeze(1), m[:, :-1]), dim=1)
    i = torch.exp(zi - m)
    f = torch.exp(zf + m_prev - m)
    z = torch.tanh(zz)
    rn = i.clone()
    rn[:, 0] = f[:, 0] * n0 + i[:, 0]
    rc = i * z
    rc[:, 0] = f[:, 0] * c0 + i[:, 0] * z[:, 0]
    n = scan_diag(f, rn)
    c = scan_diag(f, rc)
    o = torch.sigmoid(zo)
    h = o * (c / (n + eps))
    return torch.stack((c, n, m, h), dim=-2).to(dtype=out_dtype)


def picard_init(p: SLSTMParams, wx: Tensor, n_picard: int, h0: Tensor | None = None) -> Tensor:
    """Zero-hidden scan then ``n_picard`` frozen-gate passes (slstm_picard.py:160-181)."""
    states = frozen_gate_scan(wx, p.eps, h0)
    for _ in range(n_picard):
        h_prev = prepend(states, h0)[..., H, :]
        states = frozen_gate_scan(_pre(p, wx, h_prev), p.eps, h0)
    return states


def slstm_newton(
    p: SLSTMParams,
    x: Tensor,
    *,
    max_iters: int,
    picard_iters: int,
    omega: float = 1.0,
    h0: Tensor | None = None,
    wx: Tensor | None = None,
    work: str = "eager",
) -> Tensor:
    """Alg. 1 at fixed K and P (newton/__init__.py:467-549, picard.py:161-186).

    ``residual_atol=None`` semantics: all K iterations run.

    ``work='eager'`` is the reference's eager path: every op in the tensor
    dtype, states re-rounded after each update.  ``work='fused'`` is the
    semantics of the reference's fused custom op for narrow dtypes
    (kernels/newton_slstm.py:2696-2939, kernels/_fused_common.py:171-183):
    the same Picard guess (computed in the tensor dtype by the eager
    frozen-gate scan, slstm_picard.py:20-48), then every Newton iteration in
    fp32 on upcast ``wx``/``R``/``h0``, rounded to the tensor dtype once at the
    end.  For fp32 tensors the two coincide up to scan order.
    """
    if work not in ("eager", "fused"):
        raise ValueError(f"unknown work mode {work!r}")
    if wx is None:
        wx = p.wx(x)
    states = picard_init(p, wx, picard_iters, h0)
    if work == "fused" and states.dtype != torch.float32:
        out_dtype = states.dtype
        p32 = SLSTMParams(p.W.float(), p.b.float(), p.R.float(), p.eps, p.cap)
        h32 = None if h0 is None else h0.float()
        s32 = slstm_newton_iterate(p32, wx.float(), states.float(), max_iters, omega, h32)
        return s32.to(out_dtype)
    return slstm_newton_iterate(p, wx, states, max_iters, omega, h0)


def slstm_newton_iterate(p: SLSTMParams, wx: Tensor, states: Tensor, max_iters: int,
                         omega: float = 1.0, h0: Tensor | None = None) -> Tensor:
    """The K Newton updates from a given guess (newton/__init__.py:516-543)."""
    for _ in range(max_iters):
        pred, jac = slstm_jacobian(p, prepend(states, h0), wx)
        delta = scan_block4(jac, pred - states)
        if states.dtype in (torch.float16, torch.bfloat16):
            states = (states.float() + omega * delta.float()).to(states.dtype)
        else:
            states = states + omega * delta
    return states


def slstm_sequential(p: SLSTMParams, x: Tensor, h0: Tensor | None = None,
                     wx: Tensor | None = None) -> Tensor:
    """Sequential unroll with one shared input GEMM (sequential.py:61-86)."""
    if wx is None:
        wx = p.wx(x)
    state = h0 if h0 is not None else wx.new_zeros(wx.shape[0], 4, p.d)
    outs = []
    for t in range(wx.shape[1]):
        state = slstm_step(p, state, wx[:, t])
        outs.append(state)
    return torch.stack(outs, dim=1)


# ---- float64 evaluation of the same algorithm --------------------------------


def frozen_gate_scan_f64(pre: Tensor, eps: float, h0: Tensor | None = None) -> Tensor:
    """``frozen_gate_scan`` evaluated left to right in float64.

    Same recurrence as the reference's frozen-gate pass (slstm_picard.py:51-107),
    m_t = max(z_f + m_{t-1}, z_i) etc., without the fp32 cumsum: a float64
    yardstick for how far any fp32 implementation (the reference's included)
    is from the exact iterate.
    """
    q = pre.double()
    bsz, d = q.shape[0], q.shape[-1] // 4
    zi, zf, zz, zo = q.chunk(4, dim=-1)
    if h0 is None:
        c = n = m = q.new_zeros(bsz, d)
    else:
        g = h0.double()
        c, n, m = g[:, C], g[:, N], g[:, M]
    out = []
    for t in range(q.shape[1]):
        mn = torch.maximum(zf[:, t] + m, zi[:, t])
        f = torch.exp(zf[:, t] + m - mn)
        i = torch.exp(zi[:, t] - mn)
        n = f * n + i
        c = f * c + i * torch.tanh(zz[:, t])
        m = mn
        out.append(torch.stack((c, n, m, torch.sigmoid(zo[:, t]) * (c / (n + eps))), dim=-2))
    return torch.stack(out, dim=1)


def slstm_newton_f64(p: SLSTMParams, wx: Tensor, *, max_iters: int, picard_iters: int,
                     omega: float = 1.0, h0: Tensor | None = None) -> Tensor:
    """Alg. 1 at fixed K and P entirely in float64 (Picard passes included)."""
    from oracle.scan import sequential_affine

    p64 = SLSTMParams(p.W.double(), p.b.double(), p.R.double(), p.eps, p.cap)
    wx = wx.double()
    h0 = None if h0 is None else h0.double()
    states = frozen_gate_scan_f64(wx, p.eps, h0)
    for _ in range(picard_iters):
        h_prev = prepend(states, h0)[..., H, :]
        states = frozen_gate_scan_f64(_pre(p64, wx, h_prev), p.eps, h0)
    init = states
    for _ in range(max_iters):
        pred, jac = slstm_jacobian(p64, prepend(states, h0), wx)
        states = states + omega * sequential_affine(jac, pred - states, "block4")
    return init, states
