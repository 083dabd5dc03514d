"""Eq. 2.6 backward of the ParaSLSTM ``mix='diag'`` and ParaGRU ``mix='head'`` Newton
solves (test infrastructure only).

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

and, for ``ParaGRU(mix='head')``, the same generic path with the dense
per-head Jacobian (reverse dense scan ``solvers/scan.py:181-203``), the head
cell VJP ``kernels/vjp_gru.py:141-224`` with the clip masks of
``solvers/vjp.py:214-253``, and the factorised ``J^T mu`` of
``kernels/gru_head_factor.py:68-112``.

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


# ---------------------------------------------------------------------------
# ParaGRU mix='head'
# ---------------------------------------------------------------------------


def reverse_scan_dense(jac: Tensor, partial: Tensor) -> Tensor:
    """``mu`` from per-step ``J`` ``(S, T, n, n)`` ``[out, in]`` (solvers/scan.py:181-203):
    transpose, flip time, shift by one step, forward dense scan, flip back."""
    from oracle.scan import scan_dense

    j_t = jac.transpose(-1, -2)
    j_rev = j_t.new_zeros(j_t.shape)
    j_rev[:, 1:] = j_t.flip(1)[:, :-1]
    return scan_dense(j_rev.contiguous(), partial.flip(1).contiguous()).flip(1)


def gru_head_jt_mvp(h: Tensor, z: Tensor, r: Tensor, n: Tensor, a_z: Tensor, a_r: Tensor,
                    a_n: Tensor, mu: Tensor) -> Tensor:
    """``J^T mu`` at head-local gates ``(..., H, d_head)`` (kernels/gru_head_factor.py:68-112):
    ``(1-z) mu + A_z (z' (n-h) mu) + r (A_n w_n) + A_r (r' h (A_n w_n))``,
    ``w_n = n' z mu``; ``A v`` for ``(in, out)`` matrices contracts the out index."""

    def a_times(a: Tensor, v: Tensor) -> Tensor:
        return torch.matmul(a, v.unsqueeze(-1)).squeeze(-1)

    w_z = z * (1.0 - z) * ((n - h) * mu)
    g_u = a_times(a_n, (1.0 - n.square()) * (z * mu))
    return (1.0 - z) * mu + a_times(a_z, w_z) + r * g_u + a_times(a_r, r * (1.0 - r) * (h * g_u))


def gru_head_cell_vjp(h_prev: Tensor, wx: Tensor, a_z: Tensor, a_r: Tensor, a_n: Tensor,
                      mu: Tensor, work: torch.dtype = torch.float32):
    """``(g_wx (B, T, 3d), g_az, g_ar, g_an (H, d_head, d_head))`` of
    ``sum mu * f(h_prev, wx)`` (kernels/vjp_gru.py:141-224, eager head VJP): algebra
    in ``work``, outputs in ``h_prev``'s dtype."""
    dt = h_prev.dtype
    n_heads, d_head, _ = a_z.shape
    lead = h_prev.shape[:-1]
    h = h_prev.to(work).reshape(*lead, n_heads, d_head)
    m = mu.to(work).reshape(*lead, n_heads, d_head)
    az, ar, an = a_z.to(work), a_r.to(work), a_n.to(work)
    zx, rx, nx = (t.reshape(*lead, n_heads, d_head) for t in wx.to(work).chunk(3, dim=-1))

    def mix(v: Tensor, a: Tensor) -> Tensor:
        return torch.matmul(v.unsqueeze(-2), a).squeeze(-2)

    z = torch.sigmoid(mix(h, az) + zx)
    r = torch.sigmoid(mix(h, ar) + rx)
    u = h * r
    n = torch.tanh(mix(u, an) + nx)
    d_npre = m * z * (1.0 - n.square())
    d_zpre = m * (n - h) * z * (1.0 - z)
    d_u = torch.matmul(d_npre.unsqueeze(-2), an.transpose(-1, -2)).squeeze(-2)
    d_rpre = d_u * h * r * (1.0 - r)
    g_wx = torch.cat([t.reshape(*lead, n_heads * d_head) for t in (d_zpre, d_rpre, d_npre)], -1)
    g_az = torch.einsum("...hi,...ho->hio", h, d_zpre)
    g_ar = torch.einsum("...hi,...ho->hio", h, d_rpre)
    g_an = torch.einsum("...hi,...ho->hio", u, d_npre)
    return g_wx.to(dt), g_az.to(dt), g_ar.to(dt), g_an.to(dt)


def gru_head_backward(p, x: Tensor, states: Tensor, grad: Tensor, h0: Tensor | None = None,
                      work: torch.dtype = torch.float32, wx: Tensor | None = None) -> dict:
    """Gradients of ``sum(grad * H)`` for ``H = newton_apply(ParaGRU head, x)`` at
    ``H* = states`` (solvers/newton/__init__.py:765-866 generic path,
    solvers/vjp.py:214-253): dense ``J`` at ``H*``, reverse dense scan per head,
    head cell VJP, clip masks on ``A_*``, ``W_x`` VJP, ``grad h0 = J_0^T mu_0``.
    ``p`` is an ``oracle.gru_head.GRUHeadParams``.  Keys ``x, W, b, A_z, A_r, A_n``
    (+ ``h0``) and the intermediates ``mu``, ``g_wx``."""
    from oracle.gru_head import _prepend, gru_head_jacobian

    if wx is None:
        wx = p.wx(x)
    bsz, time, d = states.shape
    hh, dh = p.n_heads, p.d_head
    h_prev = _prepend(states, h0)
    _, jac = gru_head_jacobian(p, h_prev, wx)  # (B, T, H, dh, dh)
    jf = jac.permute(0, 2, 1, 3, 4).reshape(bsz * hh, time, dh, dh)
    gf = grad.reshape(bsz, time, hh, dh).permute(0, 2, 1, 3).reshape(bsz * hh, time, dh)
    mu_f = reverse_scan_dense(jf, gf)
    mu = mu_f.reshape(bsz, hh, time, dh).permute(0, 2, 1, 3).reshape(bsz, time, d)
    a_z, a_r, a_n = p.mats()
    g_wx, g_az, g_ar, g_an = gru_head_cell_vjp(h_prev, wx, a_z, a_r, a_n, mu, work)
    if p.cap is not None:
        g_az = g_az * (p.A_z.abs() <= p.cap).to(g_az.dtype)
        g_ar = g_ar * (p.A_r.abs() <= p.cap).to(g_ar.dtype)
        g_an = g_an * (p.A_n.abs() <= p.cap).to(g_an.dtype)
    gy = g_wx.reshape(-1, g_wx.shape[-1])
    xx = x.reshape(-1, x.shape[-1])
    out = {"mu": mu, "g_wx": g_wx, "x": (gy @ p.W).reshape(x.shape), "W": gy.t() @ xx,
           "b": gy.sum(0), "A_z": g_az, "A_r": g_ar, "A_n": g_an}
    if h0 is not None:
        j0 = jac[:, 0]  # (B, H, out, in)
        m0 = mu[:, 0].reshape(bsz, hh, dh)
        out["h0"] = torch.matmul(j0.transpose(-1, -2), m0.unsqueeze(-1)).squeeze(-1).reshape(bsz, d)
    return out
