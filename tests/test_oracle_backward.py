"""The CPU oracle of the eq. 2.6 backward against the reference's golden vectors
and against autograd through the sequential unroll (float64)."""

import pytest
import torch
from conftest import load_golden

from oracle.backward import reverse_scan_block4, slstm_backward, slstm_cell_vjp
from oracle.scan import sequential_affine
from oracle.slstm import SLSTMParams, slstm_newton, slstm_sequential


def _params(t, m, dtype=None):
    W, b, R = t["W"], t["b"], t["R"]
    if dtype is not None:
        W, b, R = W.to(dtype), b.to(dtype), R.to(dtype)
    return SLSTMParams(W, b, R, eps=m["eps"], cap=m["max_recurrent_norm"])


def test_bwd_parts_match_reference():
    t, m = load_golden("bwd_parts")
    mu = reverse_scan_block4(t["rev4_j"], t["rev4_p"])
    assert torch.allclose(mu, t["rev4_mu"], rtol=0, atol=2e-6)
    g_wx, g_r = slstm_cell_vjp(t["vjp_state"], t["vjp_wx"], t["vjp_r"], t["vjp_mu"], m["eps"])
    assert torch.equal(g_wx, t["vjp_gwx"])
    assert torch.allclose(g_r, t["vjp_gr"], rtol=1e-6, atol=1e-6)


def test_reverse_scan_is_the_adjoint_recursion():
    # mu_t = p_t + J_{t+1}^T mu_{t+1}, walked backwards in float64.
    g = torch.Generator().manual_seed(3)
    j = torch.randn(2, 23, 4, 4, 5, generator=g, dtype=torch.float64) * 0.5
    p = torch.randn(2, 23, 4, 5, generator=g, dtype=torch.float64)
    mu = reverse_scan_block4(j, p)
    ref = torch.empty_like(p)
    ref[:, -1] = p[:, -1]
    for t in range(21, -1, -1):
        ref[:, t] = p[:, t] + (j[:, t + 1] * ref[:, t + 1].unsqueeze(-2)).sum(dim=-3)
    assert torch.allclose(mu, ref, rtol=0, atol=1e-12)
    # and it is the transpose of the forward solve: <mu, r> = <p, delta>
    r = torch.randn(2, 23, 4, 5, generator=g, dtype=torch.float64)
    j_fwd = j.clone()
    j_fwd[:, 0] = 0
    delta = sequential_affine(j_fwd, r, "block4")
    assert torch.allclose((mu * r).sum(), (p * delta).sum(), rtol=1e-12)


@pytest.mark.parametrize("with_h0", [False, True])
def test_backward_matches_autograd_through_sequential_float64(with_h0):
    g = torch.Generator().manual_seed(11)
    B, T, d, din = 2, 40, 8, 6
    f64 = dict(dtype=torch.float64)
    W = torch.randn(4 * d, din, generator=g, **f64) * 0.3
    b = torch.randn(4 * d, generator=g, **f64) * 0.1
    R = torch.randn(4, d, generator=g, **f64) * 0.4  # some entries beyond the 0.5 clamp
    x = torch.randn(B, T, din, generator=g, **f64)
    h0 = torch.randn(B, 4, d, generator=g, **f64).abs() if with_h0 else None
    up = torch.randn(B, T, 4, d, generator=g, **f64)
    leaves = [t.clone().requires_grad_(True) for t in (x, W, b, R)]
    h0l = h0.clone().requires_grad_(True) if with_h0 else None
    H = slstm_sequential(SLSTMParams(leaves[1], leaves[2], leaves[3]), leaves[0], h0=h0l)
    grads = torch.autograd.grad((H * up).sum(), leaves + ([h0l] if with_h0 else []))
    out = slstm_backward(SLSTMParams(W, b, R), x, H.detach(), up, h0=h0, work=torch.float64)
    names = ["x", "W", "b", "R"] + (["h0"] if with_h0 else [])
    for name, ref in zip(names, grads):
        assert torch.allclose(out[name], ref, rtol=1e-10, atol=1e-10), name
    assert (R.abs() > 0.5).any() and (out["R"][R.abs() > 0.5] == 0).all()


@pytest.mark.parametrize("name", ["slstm_bwd_fp32", "slstm_bwd_bf16", "slstm_bwd_fp16"])
def test_backward_matches_reference(name):
    t, m = load_golden(name)
    dtype = getattr(torch, m["dtype"])
    p = _params(t, m)
    h0 = t.get("h0")
    x = t["x"]
    # forward: the same K, P iterate as the reference
    H = slstm_newton(p, x, max_iters=m["K"], picard_iters=m["P"], h0=h0)
    assert torch.equal(H, t["newton"])
    out = slstm_backward(p, x, t["newton"], t["grad"], h0=h0)
    for k in ["x", "W", "b", "R"] + (["h0"] if m["h0"] else []):
        ref = t[f"grad_{k}"]
        assert out[k].dtype == ref.dtype, k
        scale = ref.float().abs().max().item()
        tol = 1e-5 if dtype == torch.float32 else 0
        err = (out[k].float() - ref.float()).abs().max().item()
        assert err <= tol * max(1.0, scale), (k, err, scale)


def test_ragged_oracle_matches_reference():
    # Per-sequence solves = the reference's packed solve with J = 0 at heads.
    from oracle.gru_head import GRUHeadParams
    from oracle.ragged import (
        gru_head_newton_ragged,
        gru_head_sequential_ragged,
        slstm_newton_ragged,
        slstm_sequential_ragged,
    )

    t, m = load_golden("slstm_ragged_fp32")
    p = SLSTMParams(t["W"], t["b"], t["R"], eps=m["eps"], cap=m["max_recurrent_norm"])
    H = slstm_newton_ragged(p, t["x"], t["cu_seqlens"], max_iters=m["K"], picard_iters=m["P"],
                            h0=t["h0"])
    Hs = slstm_sequential_ragged(p, t["x"], t["cu_seqlens"], t["h0"])
    assert torch.equal(Hs, t["sequential"])
    err = ((H - t["newton"]).abs() / (1 + t["newton"].abs())).max().item()
    assert err <= 2e-5, err  # segmented vs per-sequence fp32 scan order
    t, m = load_golden("gru_head_ragged_fp32")
    p = GRUHeadParams(t["W"], t["b"], t["A_z"], t["A_r"], t["A_n"])
    H = gru_head_newton_ragged(p, t["x"], t["cu_seqlens"], max_iters=m["K"], h0=t["h0"])
    Hs = gru_head_sequential_ragged(p, t["x"], t["cu_seqlens"], t["h0"])
    assert torch.allclose(Hs, t["sequential"], rtol=0, atol=1e-6)
    assert (H - t["newton"]).abs().max().item() <= 1e-5


# ---------------------------------------------------------------------------
# ParaGRU mix='head'
# ---------------------------------------------------------------------------


def _gru_params(t, dtype=None, cap=None):
    from oracle.gru_head import GRUHeadParams

    ts = [t[k] for k in ("W", "b", "A_z", "A_r", "A_n")]
    if dtype is not None:
        ts = [v.to(dtype) for v in ts]
    return GRUHeadParams(*ts, cap=cap)


def test_gru_head_bwd_parts_match_reference():
    from oracle.backward import gru_head_cell_vjp, gru_head_jt_mvp

    t, _ = load_golden("gru_head_bwd_parts")
    jt = gru_head_jt_mvp(t["jt_h"], t["jt_z"], t["jt_r"], t["jt_n"], t["a_z"], t["a_r"],
                         t["a_n"], t["jt_mu"])
    assert torch.allclose(jt, t["jt_out"], rtol=1e-5, atol=1e-5)
    g = gru_head_cell_vjp(t["vjp_h"], t["vjp_wx"], t["a_z"], t["a_r"], t["a_n"], t["vjp_mu"])
    for mine, key in zip(g, ("vjp_gwx", "vjp_gaz", "vjp_gar", "vjp_gan")):
        assert torch.allclose(mine, t[key], rtol=1e-5, atol=1e-5), key


def test_gru_head_jt_mvp_is_dense_jacobian_transpose():
    # The factorised J^T mu equals the dense [out, in] Jacobian's transpose times mu.
    from oracle.backward import gru_head_jt_mvp
    from oracle.gru_head import GRUHeadParams, _acts, gru_head_jacobian

    g = torch.Generator().manual_seed(5)
    f64 = dict(dtype=torch.float64)
    hh, dh, d = 2, 8, 16
    p = GRUHeadParams(torch.zeros(3 * d, 1, **f64), torch.zeros(3 * d, **f64),
                      *(torch.randn(hh, dh, dh, generator=g, **f64) * 0.4 for _ in range(3)))
    h = torch.randn(3, d, generator=g, **f64)
    wx = torch.randn(3, 3 * d, generator=g, **f64)
    mu = torch.randn(3, hh, dh, generator=g, **f64)
    _, jac = gru_head_jacobian(p, h, wx)
    a = _acts(p, h, wx)
    got = gru_head_jt_mvp(a["h"], a["z"], a["r"], a["n"], p.A_z, p.A_r, p.A_n, mu)
    want = torch.matmul(jac.transpose(-1, -2), mu.unsqueeze(-1)).squeeze(-1)
    assert torch.allclose(got, want, rtol=0, atol=1e-12)


@pytest.mark.parametrize("cap", [None, 0.15])
def test_gru_head_backward_matches_autograd_float64(cap):
    from oracle.backward import gru_head_backward
    from oracle.gru_head import GRUHeadParams, gru_head_sequential

    g = torch.Generator().manual_seed(17)
    f64 = dict(dtype=torch.float64)
    B, T, hh, dh, din = 2, 30, 2, 8, 5
    d = hh * dh
    W = torch.randn(3 * d, din, generator=g, **f64) * 0.4
    b = torch.randn(3 * d, generator=g, **f64) * 0.1
    A = [torch.randn(hh, dh, dh, generator=g, **f64) * 0.3 for _ in range(3)]
    x = torch.randn(B, T, din, generator=g, **f64)
    h0 = torch.randn(B, d, generator=g, **f64) * 0.5
    up = torch.randn(B, T, d, generator=g, **f64)
    leaves = [t.clone().requires_grad_(True) for t in (x, W, b, *A, h0)]
    H = gru_head_sequential(GRUHeadParams(*leaves[1:6], cap=cap), leaves[0], h0=leaves[6])
    grads = torch.autograd.grad((H * up).sum(), leaves)
    out = gru_head_backward(GRUHeadParams(W, b, *A, cap=cap), x, H.detach(), up, h0=h0,
                            work=torch.float64)
    for name, ref in zip(["x", "W", "b", "A_z", "A_r", "A_n", "h0"], grads):
        assert torch.allclose(out[name], ref, rtol=1e-10, atol=1e-10), name
    if cap is not None:
        assert (A[0].abs() > cap).any() and (out["A_z"][A[0].abs() > cap] == 0).all()


@pytest.mark.parametrize("name", [
    "gru_head_bwd_fp32", "gru_head_bwd_bf16", "gru_head_bwd_fp16"])
def test_gru_head_backward_matches_reference(name):
    from oracle.backward import gru_head_backward
    from oracle.gru_head import gru_head_newton

    t, m = load_golden(name)
    p = _gru_params(t)
    h0 = t.get("h0")
    H = gru_head_newton(p, t["x"], max_iters=m["K"], h0=h0)
    fp32 = m["dtype"] == "float32"
    if fp32:
        assert (H - t["newton"]).abs().max().item() <= 1e-6
    else:
        assert torch.equal(H, t["newton"])
    out = gru_head_backward(p, t["x"], t["newton"], t["grad"], h0=h0)
    for k in ["x", "W", "b", "A_z", "A_r", "A_n"] + (["h0"] if m["h0"] else []):
        ref = t[f"grad_{k}"]
        assert out[k].dtype == ref.dtype, k
        scale = max(1.0, ref.float().abs().max().item())
        err = (out[k].float() - ref.float()).abs().max().item()
        assert err <= (1e-5 if fp32 else 2e-2) * scale, (k, err, scale)
