"""GPU parity of the ParaSLSTM(mix='diag') eq. 2.6 backward (HIP reverse scan
with the fused cell VJP) against the CPU oracle and the reference's golden
gradients.  Every case prints its name before running."""

import pytest
import torch
from conftest import load_golden

import oracle as O
from oracle.backward import slstm_backward

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("lookback_mode")]

DEV = "cuda:0"


def _cfg(K, P):
    from pararnn_amd import NewtonConfig

    return NewtonConfig(max_iters=K, picard_iters=P, residual_atol=None, residual_fail=None,
                        picard_adapt=False)


def _cell(t, m, dtype):
    from pararnn_amd import ParaSLSTM

    cell = ParaSLSTM(m["d_in"], m["d"], mix="diag")
    with torch.no_grad():
        cell.W_x.weight.copy_(t["W"])
        cell.W_x.bias.copy_(t["b"])
        cell.R.copy_(t["R"])
    return cell.to(device=DEV, dtype=dtype)


def _exact(t, x, states, grad, h0, wx=None):
    """The eq. 2.6 gradients in float64 at the given H* (oracle, float64 VJP);
    ``wx`` pins the projection the kernel was given."""
    p64 = O.SLSTMParams(t["W"].double(), t["b"].double(), t["R"].double())
    return slstm_backward(p64, x.double(), states.double(), grad.double(),
                          None if h0 is None else h0.double(), work=torch.float64,
                          wx=None if wx is None else wx.double())


def _exact_r_unmasked(t, x, states, grad, h0, wx=None):
    """g_r before the clamp mask: the float64 VJP with R already clamped."""
    rc = t["R"].double().clamp(-0.5, 0.5)
    p64 = O.SLSTMParams(t["W"].double(), t["b"].double(), rc, cap=None)
    return slstm_backward(p64, x.double(), states.double(), grad.double(),
                          None if h0 is None else h0.double(), work=torch.float64,
                          wx=None if wx is None else wx.double())["R"]


def _rel(got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    return ((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def _op(wx, r, h0, states, grad, eps):
    from pararnn_amd import ops

    return ops.slstm_backward_fused(wx, r, h0, states, grad, eps=eps)


def _op_vs_exact(t, m, dtype, tag, tol_wx, tol_r, tol_h0):
    """The op alone at the reference's H*: g_wx, g_r, g_h0 against float64."""
    x, states, grad = t["x"], t["newton"], t["grad"]
    h0 = t.get("h0")
    p = O.SLSTMParams(t["W"], t["b"], t["R"])
    wx = p.wx(x)
    ex = _exact(t, x, states, grad, h0, wx)
    g_wx, g_r, g_h0, g_b = _op(wx.to(DEV), p.r().to(DEV), None if h0 is None else h0.to(DEV),
                               states.to(DEV), grad.to(DEV), m["eps"])
    torch.cuda.synchronize()
    e_wx = _rel(g_wx, ex["g_wx"])
    e_r = _rel(g_r, _exact_r_unmasked(t, x, states, grad, h0, wx))
    e_b = _rel(g_b.reshape(-1), ex["b"])
    print(f"[{tag}] op vs float64: g_wx rel {e_wx:.2e}, g_r rel {e_r:.2e}, g_b rel {e_b:.2e}",
          flush=True)
    assert e_wx <= tol_wx and e_r <= tol_r and e_b <= tol_r
    if h0 is not None:
        e_h0 = _rel(g_h0, ex["h0"])
        print(f"[{tag}] g_h0 rel {e_h0:.2e}", flush=True)
        assert e_h0 <= tol_h0


def test_op_fp32_matches_float64():
    print("case bwd op fp32 (slstm_bwd_fp32 at the reference's H*)", flush=True)
    t, m = load_golden("slstm_bwd_fp32")
    _op_vs_exact(t, m, torch.float32, "fp32", 2e-5, 2e-5, 2e-5)


def test_op_bf16_matches_float64():
    # bf16 inputs widened exactly; the kernel works in fp32 and rounds g_wx to
    # bf16 once (<= 2^-9 relative per element of the largest entry).
    print("case bwd op bf16 (slstm_bwd_bf16 at the reference's H*)", flush=True)
    t, m = load_golden("slstm_bwd_bf16")
    _op_vs_exact(t, m, torch.bfloat16, "bf16", 4e-3, 1e-4, 1e-4)


def _end_to_end(name, dtype):
    from pararnn_amd import newton_apply

    t, m = load_golden(name)
    cell = _cell(t, m, dtype)
    x = t["x"].to(DEV).requires_grad_(True)
    h0 = t["h0"].to(DEV).requires_grad_(True) if "h0" in t else None
    H = newton_apply(cell, x, _cfg(m["K"], m["P"]), h0=h0)
    (H.float() * t["grad"].to(DEV).float()).sum().backward()
    got = {"x": x.grad, "W": cell.W_x.weight.grad, "b": cell.W_x.bias.grad, "R": cell.R.grad}
    if h0 is not None:
        got["h0"] = h0.grad
    return t, m, H.detach(), got


def test_autograd_fp32_matches_reference():
    print("case bwd end-to-end fp32 (newton_apply + backward vs reference grads)", flush=True)
    t, m, H, got = _end_to_end("slstm_bwd_fp32", torch.float32)
    # the same gradients in float64 at the reference's own H*
    ex = _exact(t, t["x"], t["newton"], t["grad"], t.get("h0"))
    for k, g in got.items():
        ref = t[f"grad_{k}"]
        e_ours, e_ref = _rel(g, ex[k]), _rel(ref, ex[k])
        print(f"  grad_{k}: gpu-vs-exact {e_ours:.2e}  reference-vs-exact {e_ref:.2e}  "
              f"gpu-vs-reference {_rel(g, ref):.2e}", flush=True)
        assert g.dtype == ref.dtype
        assert e_ours <= max(1e-4, 3 * e_ref), k


def test_autograd_bf16_matches_reference():
    # The bf16 gradient is ~6x more sensitive than H* itself: the fused-op
    # forward (fp32 Newton work) and the reference's eager bf16 forward land
    # 2.3% apart in H*, which moves the exact gradient by ~14%.  So parity with
    # the reference is checked at the reference's own H* (the backward alone,
    # where the reference's eager bf16 gradient is within 0.8% of float64),
    # and the end-to-end gradient against float64 at our own H*.
    from pararnn_amd.newton import _eq26_vjp

    print("case bwd end-to-end bf16 (newton_apply + backward)", flush=True)
    t, m, H, got = _end_to_end("slstm_bwd_bf16", torch.bfloat16)
    p = O.SLSTMParams(t["W"], t["b"], t["R"])
    wx = p.wx(t["x"])
    ex = _exact(t, t["x"], H.cpu(), t["grad"], None, wx)
    for k, g in got.items():
        nrel = ((g.double().cpu() - ex[k]).norm() / ex[k].norm()).item()
        print(f"  grad_{k}: norm-rel vs float64 at our H* {nrel:.3e}", flush=True)
        assert nrel <= 1e-2, k
    print("case bwd bf16 at the reference's H* vs the reference's gradients", flush=True)
    cell = _cell(t, m, torch.bfloat16)
    with torch.no_grad():
        gx, pg, _ = _eq26_vjp(cell, t["newton"].to(DEV), t["x"].to(DEV), t["grad"].to(DEV))
    names = {"R": "R", "W_x.weight": "W", "W_x.bias": "b"}
    ours = dict(x=gx, **{names[n]: g for (n, _), g in zip(cell.named_parameters(), pg)})
    for k, g in ours.items():
        ref = t[f"grad_{k}"].float()
        nrel = ((g.float().cpu() - ref).norm() / ref.norm()).item()
        print(f"  grad_{k}: norm-rel vs reference eager bf16 {nrel:.3e}", flush=True)
        assert g.dtype == torch.bfloat16 and nrel <= 2e-2, k


@pytest.mark.parametrize("B,T,d,with_h0", [
    (1, 1, 1, True), (1, 33, 5, False), (3, 129, 70, True), (2, 256, 64, False),
    (1, 1000, 130, True),
])
def test_op_ragged_shapes_fp32(B, T, d, with_h0):
    print(f"case bwd ragged B={B} T={T} d={d} h0={with_h0}", flush=True)
    g = torch.Generator().manual_seed(B * 1000 + T + d)
    din = 7
    W = torch.randn(4 * d, din, generator=g) * 0.4
    b = torch.randn(4 * d, generator=g) * 0.1
    R = torch.randn(4, d, generator=g) * 0.3
    x = torch.randn(B, T, din, generator=g)
    h0 = None
    if with_h0:
        h0 = torch.randn(B, 4, d, generator=g)
        h0[:, 1] = h0[:, 1].abs() + 0.5
    p = O.SLSTMParams(W, b, R)
    states = O.slstm_sequential(p, x, h0=h0)  # a converged H*
    grad = torch.randn(B, T, 4, d, generator=g)
    t = {"W": W, "b": b, "R": R}
    ex = _exact(t, x, states, grad, h0)
    ex_r = _exact_r_unmasked(t, x, states, grad, h0)
    g_wx, g_r, g_h0, g_b = _op(p.wx(x).to(DEV), p.r().to(DEV),
                               None if h0 is None else h0.to(DEV), states.to(DEV),
                               grad.to(DEV), 1e-6)
    e = (_rel(g_wx, ex["g_wx"]), _rel(g_r, ex_r), _rel(g_h0, ex["h0"]) if with_h0 else 0.0,
         _rel(g_b.reshape(-1), ex["b"]))
    print(f"  rel err g_wx {e[0]:.2e} g_r {e[1]:.2e} g_h0 {e[2]:.2e} g_b {e[3]:.2e}", flush=True)
    assert max(e) <= 5e-5


def test_long_sequence_bf16_cfg5_slice():
    # cfg5 shape slice: T = 32768 on 64 channels (the full d = 768 only adds
    # independent channel blocks); inputs on the solved trajectory.
    print("case bwd long bf16 T=32768 d=64", flush=True)
    g = torch.Generator().manual_seed(5)
    B, T, d, din = 1, 32768, 64, 64
    W = (torch.randn(4 * d, din, generator=g) * 0.12).to(torch.bfloat16)
    b = torch.zeros(4 * d, dtype=torch.bfloat16)
    R = (torch.randn(4, d, generator=g) * 0.06).to(torch.bfloat16)
    x = torch.randn(B, T, din, generator=g).to(torch.bfloat16)
    p = O.SLSTMParams(W, b, R)
    states = O.slstm_sequential(O.SLSTMParams(W.float(), b.float(), R.float()),
                                x.float()).to(torch.bfloat16)
    grad = torch.randn(B, T, 4, d, generator=g).to(torch.bfloat16)
    t = {"W": W.float(), "b": b.float(), "R": R.float()}
    wx = p.wx(x)
    ex = _exact(t, x.float(), states.float(), grad.float(), None, wx)
    g_wx, g_r, _, _ = _op(wx.to(DEV), p.r().to(DEV), None, states.to(DEV), grad.to(DEV), 1e-6)
    e_wx = _rel(g_wx, ex["g_wx"])
    nrel = ((g_wx.float().cpu().double() - ex["g_wx"]).norm() / ex["g_wx"].norm()).item()
    e_r = _rel(g_r, _exact_r_unmasked(t, x.float(), states.float(), grad.float(), None, wx))
    print(f"  g_wx max-rel {e_wx:.2e} norm-rel {nrel:.2e}; g_r rel {e_r:.2e}", flush=True)
    assert e_wx <= 4e-3 and nrel <= 4e-3 and e_r <= 1e-3


def test_cfg5_gradients_on_finite_channel_slice():
    """BASELINE config 5 as timed (ParaSLSTM diag d=768, B=4, T=32768, bf16,
    K=2, P=5, x and dL/dH ~ N(0, 1), default seeded init): the eq. 2.6
    backward of the GPU's own H*.  At these pinned K, P the reference's
    algorithm leaves its basin on some channels (H* non-finite there; the
    bench line reports the fraction), so the value check runs on channels
    whose H* is finite.  Channels are independent in the diagonal Jacobian,
    so dL/dwx and the R / bias gradients of a channel depend only on that
    channel's wx, H* and dL/dH: the float64 oracle re-derives them on the
    slice."""
    from pararnn_amd import NewtonConfig, ParaSLSTM, newton_apply, ops

    print("case cfg5 gradients on a finite channel slice (d=768 B=4 T=32768 bf16)", flush=True)
    b5, t5, d5 = 4, 32768, 768
    torch.manual_seed(0)
    cell = ParaSLSTM(d5, d5).to(DEV, torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(b5, t5, d5, generator=g, device=DEV).to(torch.bfloat16)
    up = torch.randn(b5, t5, 4, d5, generator=g, device=DEV).to(torch.bfloat16)
    cfg = NewtonConfig(max_iters=2, picard_iters=5, residual_atol=None, residual_fail=None,
                       picard_adapt=False)
    with torch.no_grad():
        wx = cell.W_x(x)
        H = newton_apply(cell, x, cfg)
        r = cell.clipped_r()
        g_wx, g_r, _, g_b = ops.slstm_backward_fused(wx, r, None, H, up, eps=cell.eps)
        finite = torch.isfinite(H.float()).all(dim=(0, 1, 2)).cpu()
    frac_bad = 1.0 - finite.double().mean().item()
    ok = torch.nonzero(finite).flatten()
    print(f"  non-finite H* channels: {int((~finite).sum())} of {d5} ({frac_bad:.3f})", flush=True)
    assert ok.numel() >= 8
    chans = ok[torch.linspace(0, ok.numel() - 1, 8).round().long()]
    idx = torch.cat([chans + gi * d5 for gi in range(4)]).to(DEV)
    cd = chans.to(DEV)
    wx_s = wx[:, :, idx].cpu()
    H_s = H[:, :, :, cd].cpu()
    up_s = up[:, :, :, cd].cpu()
    R_s = cell.R.detach()[:, cd].cpu()
    t = {"W": torch.zeros(4 * 8, 1, dtype=torch.float64),
         "b": torch.zeros(4 * 8, dtype=torch.float64), "R": R_s.double()}
    dummy_x = torch.zeros(b5, t5, 1, dtype=torch.float64)
    ex = _exact(t, dummy_x, H_s.float(), up_s.float(), None, wx_s.float())
    ex_r = _exact_r_unmasked(t, dummy_x, H_s.float(), up_s.float(), None, wx_s.float())
    got_wx = g_wx[:, :, idx].cpu()
    e_wx = _rel(got_wx, ex["g_wx"])
    n_wx = ((got_wx.double() - ex["g_wx"]).norm() / ex["g_wx"].norm()).item()
    e_r = _rel(g_r[:, cd], ex_r)
    e_b = _rel(g_b.reshape(4, d5)[:, cd].reshape(-1), ex["b"])
    print(f"  channels {chans.tolist()}: g_wx max-rel {e_wx:.2e} norm-rel {n_wx:.2e}, "
          f"g_r rel {e_r:.2e}, g_b rel {e_b:.2e}", flush=True)
    assert e_wx <= 4e-3 and n_wx <= 4e-3 and e_r <= 1e-3 and e_b <= 1e-3
