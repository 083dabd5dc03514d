"""Eager affine-monoid scans (restates reference ``solvers/scan.py``).

Solves ``delta_t = J_t delta_{t-1} + r_t`` with ``delta_{-1} = 0`` along the
time axis (dim 1).  The reference uses a work-efficient Blelloch exclusive
scan, padded to a power of two with the identity ``(I, 0)``, in fp32 when the
tensors are fp16/bf16 (``scan.py:229-246, 298-323, 351-377``).  The result
is rounded back to the input dtype.
"""

from __future__ import annotations

import torch
from torch import Tensor

# ---- per-structure monoid pieces (scan.py:380-465) -------------------------


def _mv4(j: Tensor, v: Tensor) -> Tensor:
    # (..., out, in, d) x (..., in, d) -> (..., out, d); scan.py:445-447
    return (j * v.unsqueeze(-3)).sum(dim=-2)


def _mm4(a: Tensor, b: Tensor) -> Tensor:
    # a @ b per channel, reduce over the inner index; scan.py:450-452
    return (a.unsqueeze(-2) * b.unsqueeze(-4)).sum(dim=-3)


def _ident4(slot: Tensor) -> None:
    slot.zero_()
    for k in range(4):
        slot[..., k, k, :] = 1


def _ident_dense(slot: Tensor) -> None:
    slot.zero_()
    slot.diagonal(dim1=-2, dim2=-1).fill_(1)


def _ident_diag(slot: Tensor) -> None:
    slot.fill_(1.0)


_OPS = {
    # name: (compose(right, left), apply(J, v), identity fill)
    "diag": (lambda jr, rr, jl, rl: (jr * jl, jr * rl + rr), lambda j, v: j * v, _ident_diag),
    "block4": (
        lambda jr, rr, jl, rl: (_mm4(jr, jl), _mv4(jr, rl) + rr),
        _mv4,
        _ident4,
    ),
    "dense": (
        lambda jr, rr, jl, rl: (jr @ jl, (jr @ rl.unsqueeze(-1)).squeeze(-1) + rr),
        lambda j, v: (j @ v.unsqueeze(-1)).squeeze(-1),
        _ident_dense,
    ),
}


def blelloch_inclusive(jac: Tensor, res: Tensor, kind: str) -> Tensor:
    """Inclusive solve by up-sweep / down-sweep (scan.py:298-323, 351-377).

    Works in the dtype it is given (callers upcast).  The up-sweep composes
    ``right <- right (+) left`` at stride 2^k; the root is reset to the
    identity; the down-sweep swaps the left child into place and composes
    the parent prefix *before* the left subtree.  The inclusive value at t is
    ``J_t * prefix_t + r_t``.
    """
    compose, apply, ident = _OPS[kind]
    time = res.shape[1]
    if time <= 1:
        return res.clone()
    n = 1 << (time - 1).bit_length()
    j = jac.new_empty(jac.shape[0], n, *jac.shape[2:])
    r = res.new_empty(res.shape[0], n, *res.shape[2:])
    j[:, :time] = jac
    r[:, :time] = res
    if n > time:
        ident(j[:, time:])
        r[:, time:] = 0
    stride = 2
    while stride <= n:
        hi = torch.arange(stride - 1, n, stride)
        lo = hi - stride // 2
        j[:, hi], r[:, hi] = compose(j[:, hi], r[:, hi], j[:, lo], r[:, lo])
        stride *= 2
    ident(j[:, n - 1])
    r[:, n - 1] = 0
    stride = n
    while stride >= 2:
        hi = torch.arange(stride - 1, n, stride)
        lo = hi - stride // 2
        j_lo = j[:, lo].clone()
        r_lo = r[:, lo].clone()
        j[:, lo] = j[:, hi]
        r[:, lo] = r[:, hi]
        j[:, hi], r[:, hi] = compose(j_lo, r_lo, j[:, hi], r[:, hi])
        stride //= 2
    return apply(jac, r[:, :time]) + res


def _acc(jac: Tensor, res: Tensor, kind: str) -> Tensor:
    # scan.py:229-246: fp32 algebra for narrow dtypes, result in the input dtype
    if jac.dtype in (torch.float16, torch.bfloat16):
        return blelloch_inclusive(jac.float(), res.float(), kind).to(jac.dtype)
    return blelloch_inclusive(jac, res, kind)


def scan_diag(jac: Tensor, res: Tensor) -> Tensor:
    """``(B,T,d)`` diagonal J (scan.py:31-57, eager branch)."""
    return _acc(jac, res, "diag")


def scan_block4(jac: Tensor, res: Tensor) -> Tensor:
    """``(B,T,4,4,d)`` ``[..., out, in, d]`` J, ``(B,T,4,d)`` r (scan.py:82-100)."""
    return _acc(jac, res, "block4")


def scan_dense(jac: Tensor, res: Tensor) -> Tensor:
    """``(B,T,n,n)`` ``[..., out, in]`` J, ``(B,T,n)`` r (scan.py:103-123)."""
    return _acc(jac, res, "dense")


def sequential_affine(jac: Tensor, res: Tensor, kind: str) -> Tensor:
    """Brute-force left-to-right recurrence; the invariant every scan must meet."""
    _, apply, _ = _OPS[kind]
    out = torch.empty_like(res)
    delta = torch.zeros_like(res[:, 0])
    for t in range(res.shape[1]):
        delta = apply(jac[:, t], delta) + res[:, t]
        out[:, t] = delta
    return out
