"""ParaGRU ``mix='head'`` eager restatement (test infrastructure only).

Restates, on the CPU:
* the head cell — reference ``cells/para_gru.py:443-467`` (``_recurrence``,
  head branch) with ``(in, out)`` recurrent matrices per head;
* the dense per-head Jacobian — ``cells/para_gru.py:385-412``;
* App. A initial guess ``f(h_prev0, x_t)`` with ``h_prev0`` zero except
  ``h0`` at t = 0 — ``solvers/newton/__init__.py:925-940, 481-494``;
* the eager Newton loop and the head slot pack into a dense Blelloch scan —
  ``solvers/newton/__init__.py:516-543``, ``solvers/newton/dispatch.py:292-300,
  455-507``, ``solvers/scan.py:103-123``;
* the sequential unroll — ``solvers/sequential.py:22-86``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor

from oracle.scan import scan_dense


@dataclass
class GRUHeadParams:
    W: Tensor  # (3d, d_in)
    b: Tensor  # (3d,)
    A_z: Tensor  # (H, d_head, d_head), (in, out)
    A_r: Tensor
    A_n: Tensor
    cap: float | None = None

    @property
    def n_heads(self) -> int:
        return self.A_z.shape[0]

    @property
    def d_head(self) -> int:
        return self.A_z.shape[-1]

    @property
    def d(self) -> int:
        return self.n_heads * self.d_head

    def mats(self) -> tuple[Tensor, Tensor, Tensor]:
        # para_gru.py:252-281 (no clamp unless a cap is set)
        if self.cap is None:
            return self.A_z, self.A_r, self.A_n
        c = self.cap
        return self.A_z.clamp(-c, c), self.A_r.clamp(-c, c), self.A_n.clamp(-c, c)

    def wx(self, x: Tensor) -> Tensor:
        return F.linear(x, self.W, self.b)


def _mix(hv: Tensor, a: Tensor) -> Tensor:
    # h @ A per head (para_gru.py:414-416)
    return torch.matmul(hv.unsqueeze(-2), a).squeeze(-2)


def _acts(p: GRUHeadParams, h: Tensor, wx: Tensor) -> dict:
    a_z, a_r, a_n = p.mats()
    lead = h.shape[:-1]
    hv = h.reshape(*lead, p.n_heads, p.d_head)
    zx, rx, nx = (t.reshape(*lead, p.n_heads, p.d_head) for t in wx.chunk(3, dim=-1))
    z = torch.sigmoid(_mix(hv, a_z) + zx)
    r = torch.sigmoid(_mix(hv, a_r) + rx)
    n = torch.tanh(_mix(hv * r, a_n) + nx)
    new = torch.lerp(hv, n, z).reshape(*lead, p.d)
    return dict(h=hv, z=z, r=r, n=n, new=new, a=(a_z, a_r, a_n))


def gru_head_step(p: GRUHeadParams, h: Tensor, wx: Tensor) -> Tensor:
    return _acts(p, h, wx)["new"]


def gru_head_jacobian(p: GRUHeadParams, h: Tensor, wx: Tensor) -> tuple[Tensor, Tensor]:
    """``(f(h), J)`` with J ``(..., H, d_head, d_head)`` laid out ``[out, in]``."""
    a = _acts(p, h, wx)
    hv, z, r, n = a["h"], a["z"], a["r"], a["n"]
    a_z, a_r, a_n = a["a"]
    eye = torch.eye(p.d_head, dtype=h.dtype)
    zp = z * (1.0 - z)
    rp = r * (1.0 - r)
    np_ = 1.0 - n.square()
    dz = zp.unsqueeze(-1) * a_z.transpose(-1, -2)
    dr = rp.unsqueeze(-1) * a_r.transpose(-1, -2)
    du = torch.add(hv.unsqueeze(-1) * dr, r.unsqueeze(-1) * eye)
    dn = torch.matmul(np_.unsqueeze(-1) * a_n.transpose(-1, -2), du)
    jac = (1.0 - z).unsqueeze(-1) * eye + (n - hv).unsqueeze(-1) * dz + z.unsqueeze(-1) * dn
    return a["new"], jac


def _prepend(states: Tensor, h0: Tensor | None) -> Tensor:
    out = states.new_empty(states.shape)
    out[:, 0] = 0 if h0 is None else h0
    out[:, 1:] = states[:, :-1]
    return out


def _head_scan(p: GRUHeadParams, jac: Tensor, res: Tensor) -> Tensor:
    # dispatch.py:455-507: fold heads into the batch, dense scan, unfold
    bsz, time = res.shape[:2]
    hh, dh = p.n_heads, p.d_head
    jf = jac.permute(0, 2, 1, 3, 4).reshape(bsz * hh, time, dh, dh).contiguous()
    rf = res.reshape(bsz, time, hh, dh).permute(0, 2, 1, 3).reshape(bsz * hh, time, dh)
    delta = scan_dense(jf, rf.contiguous())
    return delta.reshape(bsz, hh, time, dh).permute(0, 2, 1, 3).reshape(bsz, time, hh * dh)


def gru_head_newton(
    p: GRUHeadParams,
    x: Tensor,
    *,
    max_iters: int,
    omega: float = 1.0,
    h0: Tensor | None = None,
    wx: Tensor | None = None,
    work: str = "eager",
) -> Tensor:
    """Alg. 1 at fixed K (newton/__init__.py:467-549).

    ``work='fused'`` is the semantics of the reference's fused head op for
    narrow dtypes (kernels/newton_gru_head.py:655-717): ``wx``, ``A_*`` and
    ``h0`` upcast to fp32, the initial guess and all K iterations in fp32,
    one rounding to the tensor dtype at the end.
    """
    if work not in ("eager", "fused"):
        raise ValueError(f"unknown work mode {work!r}")
    if wx is None:
        wx = p.wx(x)
    if work == "fused" and wx.dtype != torch.float32:
        p32 = GRUHeadParams(p.W.float(), p.b.float(), p.A_z.float(), p.A_r.float(),
                            p.A_n.float(), p.cap)
        out = gru_head_newton(p32, x, max_iters=max_iters, omega=omega,
                              h0=None if h0 is None else h0.float(), wx=wx.float())
        return out.to(wx.dtype)
    bsz, time = wx.shape[:2]
    h_prev0 = wx.new_zeros(bsz, time, p.d)
    if h0 is not None:
        h_prev0[:, 0] = h0
    states = gru_head_step(p, h_prev0, wx)
    for _ in range(max_iters):
        pred, jac = gru_head_jacobian(p, _prepend(states, h0), wx)
        delta = _head_scan(p, jac, pred - states)
        if states.dtype in (torch.float16, torch.bfloat16):
            states = (states.float() + omega * delta.float()).to(states.dtype)
        else:
            states = states + omega * delta
    return states


def gru_head_sequential(p: GRUHeadParams, x: Tensor, h0: Tensor | None = None,
                        wx: Tensor | None = None) -> Tensor:
    if wx is None:
        wx = p.wx(x)
    h = h0 if h0 is not None else wx.new_zeros(wx.shape[0], p.d)
    outs = []
    for t in range(wx.shape[1]):
        h = gru_head_step(p, h, wx[:, t])
        outs.append(h)
    return torch.stack(outs, dim=1)
