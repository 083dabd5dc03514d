"""Eq. 2.6 backward of the ParaSLSTM ``mix='diag'`` Newton solve (test infrastructure only).

Restates, on the CPU:
* the implicit-function backward ``_eq26_vjp`` — reference
  ``solvers/newton/__init__.py:765-866`` (generic path: Jacobian at ``H*``,
  reverse scan, packed cell VJP, ``h0`` adjoint ``J_0^T mu_0``);
* the reverse 4x4 scan — ``solvers/scan.py:166-178`` (``J^T``, time flip,
  shift by one step, forward ``scan_block4``, flip back);
* the packed channelwise cell VJP — ``kernels/vjp_slstm.py:173-240``
  (``slstm_recurrence_vjp_eager``: fp32 algebra, output in ``wx``'s dtype);
* the clip mask and the ``W_x`` VJP — ``solvers/vjp.py:103-120, 288-306``;
* the ``h0`` adjoint — ``solvers/newton/dispatch.py:406-410``.

The adjoint recursion is ``mu_{T-1} = g_{T-1}``,
``mu_t = g_t + J_{t+1}^T mu_{t+1}``; ``grad h0 = J_0^T mu_0``.
"""

from __future__ import annotations

import torch
from torch import Tensor

from oracle.scan import scan_block4
from oracle.slstm import C, H, M, N, SLSTMParams, prepend, slstm_jacobian


def reverse_scan_block4(jac: Tensor, partial: Tensor) -> Tensor:
    """``mu`` from ``J`` ``(B, T, 4, 4, d)`` ``[out, in, d]`` and ``partial`` (scan.py:166-178)."""
    j_t = jac.transpose(-3, -2)
    j_rev = j_t.new_zeros(j_t.shape)
    j_rev[:, 1:] = j_t.flip(1)[:, :-1]
    return scan_block4(j_rev, partial.flip(1)).flip(1)


def slstm_cell_vjp(state_prev: Tensor, wx: Tensor, r: Tensor, mu: Tensor, eps: float,
                   work: torch.dtype = torch.float32) -> tuple[Tensor, Tensor]:
    """``(g_wx (B, T, 4d), g_r (4, d))`` of ``sum mu * f(state_prev, wx)`` (vjp_slstm.py:173-240).

    The reference evaluates in fp32 (``work``); float64 is for pinning.
    """
    dt = wx.dtype
    rdt = r.dtype
    sp = state_prev.to(work)
    wx = wx.to(work)
    r = r.to(work)
    mu = mu.to(work)
    c_prev, n_prev, m_prev, h_prev = sp[..., C, :], sp[..., N, :], sp[..., M, :], sp[..., H, :]
    mu_c, mu_n, mu_m, mu_h = mu[..., C, :], mu[..., N, :], mu[..., M, :], mu[..., H, :]
    wx_i, wx_f, wx_z, wx_o = wx.chunk(4, dim=-1)
    r_i, r_f, r_z, r_o = r.unbind(0)
    z_i = wx_i + r_i * h_prev
    z_f = wx_f + r_f * h_prev
    z_z = wx_z + r_z * h_prev
    z_o = wx_o + r_o * h_prev
    left = z_f + m_prev
    m_new = torch.maximum(left, z_i)
    alpha = (left > z_i).to(left.dtype) + 0.5 * (left == z_i).to(left.dtype)
    i_t = torch.exp(z_i - m_new)
    f_t = torch.exp(z_f + m_prev - m_new)
    z = torch.tanh(z_z)
    n_new = f_t * n_prev + i_t
    c_new = f_t * c_prev + i_t * z
    o = torch.sigmoid(z_o)
    denom = n_new + eps
    d_o = mu_h * (c_new / denom)
    d_cnew = mu_c + mu_h * (o / denom)
    d_nnew = mu_n + mu_h * (-o * c_new / denom.square())
    d_f = d_cnew * c_prev + d_nnew * n_prev
    d_i = d_cnew * z + d_nnew
    d_z = d_cnew * i_t
    d_zo = d_o * o * (1.0 - o)
    d_zz = d_z * (1.0 - z.square())
    d_mnew = mu_m - d_i * i_t - d_f * f_t
    d_zi = d_i * i_t + d_mnew * (1.0 - alpha)
    d_zf = d_f * f_t + d_mnew * alpha
    g_wx = torch.cat((d_zi, d_zf, d_zz, d_zo), dim=-1)
    dims = (0, 1)
    g_r = torch.stack([(g * h_prev).sum(dim=dims) for g in (d_zi, d_zf, d_zz, d_zo)], dim=0)
    return g_wx.to(dt), g_r.to(rdt)


def slstm_backward(p: SLSTMParams, x: Tensor, states: Tensor, grad: Tensor,
                   h0: Tensor | None = None, work: torch.dtype = torch.float32,
                   wx: Tensor | None = None) -> dict:
    """Gradients of ``sum(grad * H)`` for ``H = newton_apply(cell, x)`` at ``H* = states``.

    Returns ``x``, ``W``, ``b``, ``R`` and (when ``h0`` is given) ``h0``
    gradients plus the intermediates ``mu`` and ``g_wx``, every tensor in the
    dtype the reference produces it in.  ``wx`` overrides ``W_x(x)`` (to
    evaluate at exactly the projection a caller used).
    """
    if wx is None:
        wx = p.wx(x)
    h_prev = prepend(states, h0)
    _, jac = slstm_jacobian(p, h_prev, wx)
    mu = reverse_scan_block4(jac, grad)
    g_wx, g_r = slstm_cell_vjp(h_prev, wx, p.r(), mu, p.eps, work)
    if p.cap is not None:
        g_r = g_r * (p.R.abs() <= p.cap).to(g_r.dtype)
    gy = g_wx.reshape(-1, g_wx.shape[-1])
    xx = x.reshape(-1, x.shape[-1])
    out = {
        "mu": mu,
        "g_wx": g_wx,
        "x": (gy @ p.W).reshape(x.shape),
        "W": gy.t() @ xx,
        "b": gy.sum(0),
        "R": g_r,
    }
    if h0 is not None:
        # J_0^T mu_0 per channel: sum over the out index
        out["h0"] = (jac[:, 0] * mu[:, 0].unsqueeze(-2)).sum(dim=-3)
    return out
