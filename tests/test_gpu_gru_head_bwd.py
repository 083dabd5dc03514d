"""GPU parity of the ParaGRU(mix='head') eq. 2.6 backward (chunked reverse
scan with Phi^T carries, fused head cell VJP, MFMA dL/dA reduction) against
the reference's golden vectors, the CPU oracle and float64 autograd.  Every
case prints its name before running."""

import pytest
import torch
from conftest import load_golden

from oracle.backward import gru_head_backward
from oracle.gru_head import GRUHeadParams, gru_head_sequential

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _cfg(K):
    from pararnn_amd import NewtonConfig

    return NewtonConfig(max_iters=K, residual_atol=None, residual_fail=None)


def _params(t):
    return GRUHeadParams(t["W"], t["b"], t["A_z"], t["A_r"], t["A_n"])


def _cell_from(t, m, dtype):
    from pararnn_amd import ParaGRU

    cell = ParaGRU(m["d_in"], m["d"], mix="head", n_heads=m["n_heads"])
    with torch.no_grad():
        cell.W_x.weight.copy_(t["W"])
        cell.W_x.bias.copy_(t["b"])
        for k in ("A_z", "A_r", "A_n"):
            getattr(cell, k).copy_(t[k])
    return cell.to(device=DEV, dtype=dtype)


def _op(p, x, states, grad, h0, dtype):
    from pararnn_amd import ops

    wx = p.wx(x.float()).to(dtype) if dtype == torch.float32 else p.wx(x)
    a = [t.to(DEV, dtype) for t in p.mats()]
    g_wx, g_a, g_h0 = ops.gru_head_backward_fused(
        wx.to(DEV), *a, None if h0 is None else h0.to(DEV, dtype), states.to(DEV, dtype),
        grad.to(DEV, dtype))
    return wx, g_wx.cpu(), g_a.cpu(), g_h0.cpu()


def _rel(a, b):
    return ((a.float() - b.float()).abs().max() / b.float().abs().max().clamp_min(1e-30)).item()


def test_op_at_reference_trajectory_fp32(walk_kernel):
    print("case gru_head_bwd_fp32 op at reference H*", flush=True)
    t, m = load_golden("gru_head_bwd_fp32")
    p = _params(t)
    wx, g_wx, g_a, g_h0 = _op(p, t["x"], t["newton"], t["grad"], t["h0"], torch.float32)
    ref = gru_head_backward(p, t["x"], t["newton"], t["grad"], h0=t["h0"], wx=wx)
    errs = {"g_wx": _rel(g_wx, ref["g_wx"]), "h0": _rel(g_h0, ref["h0"])}
    for i, k in enumerate(("A_z", "A_r", "A_n")):
        errs[k] = _rel(g_a[i], ref[k])
    print("  rel err " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v <= 1e-5, k


def test_autograd_matches_reference_grads_fp32():
    from pararnn_amd import newton_apply

    print("case gru_head_bwd_fp32 end to end vs reference grads", flush=True)
    t, m = load_golden("gru_head_bwd_fp32")
    cell = _cell_from(t, m, torch.float32)
    x = t["x"].to(DEV).requires_grad_(True)
    h0 = t["h0"].to(DEV).requires_grad_(True)
    H = newton_apply(cell, x, _cfg(m["K"]), h0=h0)
    (H * t["grad"].to(DEV)).sum().backward()
    got = {"x": x.grad, "h0": h0.grad, "W": cell.W_x.weight.grad, "b": cell.W_x.bias.grad,
           "A_z": cell.A_z.grad, "A_r": cell.A_r.grad, "A_n": cell.A_n.grad}
    for k, g in got.items():
        e = _rel(g.cpu(), t[f"grad_{k}"])
        print(f"  {k}: rel err {e:.2e}", flush=True)
        assert e <= 1e-4, k


def test_op_at_reference_trajectory_bf16(walk_kernel):
    print("case gru_head_bwd_bf16 op at reference H*", flush=True)
    t, m = load_golden("gru_head_bwd_bf16")
    p = _params(t)
    wx, g_wx, g_a, _ = _op(p, t["x"], t["newton"], t["grad"], None, torch.bfloat16)
    # fp32 algebra on the bf16 operands, as the op computes
    p32 = GRUHeadParams(*(v.float() for v in (p.W, p.b, p.A_z, p.A_r, p.A_n)))
    ref = gru_head_backward(p32, t["x"].float(), t["newton"].float(), t["grad"].float(),
                            wx=wx.float())
    errs = {"g_wx": _rel(g_wx, ref["g_wx"])}
    for i, k in enumerate(("A_z", "A_r", "A_n")):
        errs[k] = _rel(g_a[i], ref[k])
    print("  rel err " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v <= 2e-2, k
    # and the reference's own bf16 gradients, through the W_x VJP
    gy = g_wx.float().reshape(-1, g_wx.shape[-1])
    e = _rel(gy.t() @ t["x"].float().reshape(-1, t["x"].shape[-1]), t["grad_W"])
    print(f"  W vs reference bf16 grad: rel err {e:.2e}", flush=True)
    assert e <= 3e-2


@pytest.fixture(params=["vec", "mfma"])
def walk_kernel(request, monkeypatch):
    """Run with each reverse-walk kernel (per-lane mat-vecs / matrix cores)."""
    monkeypatch.setenv("PRNN_GRU_REV_MFMA", "1" if request.param == "mfma" else "0")
    return request.param


@pytest.mark.parametrize("B,T,H,with_h0", [(1, 1, 1, True), (2, 33, 1, False),
                                           (2, 1000, 4, True), (1, 4096, 2, True),
                                           (1, 1700, 1, True)])
def test_op_vs_oracle_float64(B, T, H, with_h0, walk_kernel):
    print(f"case op vs float64 oracle B={B} T={T} H={H} h0={with_h0} walks={walk_kernel}",
          flush=True)
    g = torch.Generator().manual_seed(B * 7 + T + H)
    d, din = 64 * H, 24
    p = GRUHeadParams(torch.randn(3 * d, din, generator=g) * 0.2, torch.randn(3 * d, generator=g) * 0.1,
                      *(torch.randn(H, 64, 64, generator=g) * 0.15 for _ in range(3)))
    x = torch.randn(B, T, din, generator=g)
    h0 = torch.randn(B, d, generator=g) * 0.5 if with_h0 else None
    states = torch.tanh(torch.randn(B, T, d, generator=g))
    grad = torch.randn(B, T, d, generator=g)
    wx, g_wx, g_a, g_h0 = _op(p, x, states, grad, h0, torch.float32)
    p64 = GRUHeadParams(*(v.double() for v in (p.W, p.b, p.A_z, p.A_r, p.A_n)))
    ref = gru_head_backward(p64, x.double(), states.double(), grad.double(),
                            h0=None if h0 is None else h0.double(), work=torch.float64,
                            wx=wx.double())
    errs = {"g_wx": _rel(g_wx, ref["g_wx"])}
    for i, k in enumerate(("A_z", "A_r", "A_n")):
        errs[k] = _rel(g_a[i], ref[k])
    if with_h0:
        errs["h0"] = _rel(g_h0, ref["h0"])
    print("  rel err " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v <= 2e-5, k


def test_end_to_end_vs_float64_autograd_of_sequential():
    from pararnn_amd import ParaGRU, newton_apply

    print("case end-to-end grads vs float64 autograd through the sequential unroll", flush=True)
    torch.manual_seed(3)
    B, T, H, din = 2, 300, 2, 16
    cell = ParaGRU(din, 64 * H, mix="head", n_heads=H).to(DEV)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, T, din, generator=g)
    h0 = torch.randn(B, 64 * H, generator=g) * 0.5
    up = torch.randn(B, T, 64 * H, generator=g)
    xd = x.to(DEV).requires_grad_(True)
    hd = h0.to(DEV).requires_grad_(True)
    (newton_apply(cell, xd, _cfg(8), h0=hd) * up.to(DEV)).sum().backward()
    leaves = [v.detach().cpu().double().requires_grad_(True) for v in
              (cell.W_x.weight, cell.W_x.bias, cell.A_z, cell.A_r, cell.A_n)]
    x64 = x.double().requires_grad_(True)
    h64 = h0.double().requires_grad_(True)
    Hs = gru_head_sequential(GRUHeadParams(*leaves), x64, h0=h64)
    ref = torch.autograd.grad((Hs * up.double()).sum(), [x64, h64, *leaves])
    got = [xd.grad, hd.grad, cell.W_x.weight.grad, cell.W_x.bias.grad, cell.A_z.grad,
           cell.A_r.grad, cell.A_n.grad]
    for name, a, b in zip(["x", "h0", "W", "b", "A_z", "A_r", "A_n"], got, ref):
        e = _rel(a.cpu().double(), b)
        print(f"  {name}: rel err {e:.2e}", flush=True)
        assert e <= 1e-4, name


def test_full_length_linearity_and_one_head_slice():
    """cfg4's T at B=1: the op is linear in the upstream gradient, and head 0
    alone (heads never mix) matches the fp32 oracle on its own parameters."""
    print("case full-length T=32768 H=8: linearity + head-0 slice vs oracle", flush=True)
    g = torch.Generator().manual_seed(11)
    B, T, H, din = 1, 32768, 8, 32
    d = 64 * H
    p = GRUHeadParams(torch.randn(3 * d, din, generator=g) * 0.2, torch.randn(3 * d, generator=g) * 0.1,
                      *(torch.randn(H, 64, 64, generator=g) * 0.15 for _ in range(3)))
    x = torch.randn(B, T, din, generator=g)
    states = torch.tanh(torch.randn(B, T, d, generator=g))
    g1 = torch.randn(B, T, d, generator=g)
    g2 = torch.randn(B, T, d, generator=g)
    _, a_wx, a_a, _ = _op(p, x, states, g1, None, torch.float32)
    _, b_wx, b_a, _ = _op(p, x, states, g2, None, torch.float32)
    _, c_wx, c_a, _ = _op(p, x, states, g1 + 2 * g2, None, torch.float32)
    e_lin = max(_rel(c_wx, a_wx + 2 * b_wx), _rel(c_a, a_a + 2 * b_a))
    print(f"  linearity rel err {e_lin:.2e}", flush=True)
    assert e_lin <= 1e-5
    rows = torch.cat([torch.arange(64) + k * d for k in range(3)])
    p0 = GRUHeadParams(p.W[rows], p.b[rows], p.A_z[:1], p.A_r[:1], p.A_n[:1])
    ref = gru_head_backward(p0, x, states[..., :64], g1[..., :64])
    e_wx = _rel(a_wx.reshape(B, T, 3, H, 64)[:, :, :, 0].reshape(B, T, 192), ref["g_wx"])
    e_a = max(_rel(a_a[i, 0], ref[k]) for i, k in enumerate(("A_z", "A_r", "A_n")))
    print(f"  head 0 vs oracle: g_wx {e_wx:.2e} g_a {e_a:.2e}", flush=True)
    assert e_wx <= 1e-4 and e_a <= 1e-4


def test_recompute_chunk_len_and_packed_sequences():
    """The other autograd routes of newton_apply: recompute (bit-equal), chunk_len
    windows and packed cu_seqlens (equal to per-sequence solves)."""
    from pararnn_amd import NewtonConfig, ParaGRU, newton_apply

    print("case head GRU grads: recompute, chunk_len, cu_seqlens", flush=True)
    torch.manual_seed(6)
    cell = ParaGRU(12, 128, mix="head", n_heads=2).to(DEV)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 150, 12, generator=g).to(DEV)
    h0 = (torch.randn(2, 128, generator=g) * 0.5).to(DEV)
    up = torch.randn(2, 150, 128, generator=g).to(DEV)

    def grads(cfg, **kw):
        cell.zero_grad()
        xx = x.clone().requires_grad_(True)
        hh = h0.clone().requires_grad_(True)
        (newton_apply(cell, xx, cfg, h0=hh, **kw) * up).sum().backward()
        return [xx.grad, hh.grad] + [p.grad.clone() for p in cell.parameters()]

    base = NewtonConfig(max_iters=8, residual_atol=None, residual_fail=None)
    ref = grads(base)
    rec = grads(NewtonConfig(max_iters=8, residual_atol=None, residual_fail=None, recompute=True))
    for a, b in zip(ref, rec):
        assert torch.equal(a, b)
    chk = grads(NewtonConfig(max_iters=8, residual_atol=None, residual_fail=None, chunk_len=64))
    for a, b in zip(ref, chk):
        e = _rel(b.cpu(), a.cpu())
        assert e <= 1e-4, e
    # packed: two sequences of the batch laid end to end
    cell.zero_grad()
    xp = torch.cat([x[0], x[1, :90]], 0).unsqueeze(0).clone().requires_grad_(True)
    hp = h0.clone().requires_grad_(True)
    upp = torch.cat([up[0], up[1, :90]], 0).unsqueeze(0)
    cs = torch.tensor([0, 150, 240], device=DEV)
    (newton_apply(cell, xp, base, h0=hp, cu_seqlens=cs) * upp).sum().backward()
    packed = [p.grad.clone() for p in cell.parameters()]
    cell.zero_grad()
    xs = [x[0:1].clone().requires_grad_(True), x[1:2, :90].clone().requires_grad_(True)]
    hs = h0.clone().requires_grad_(True)
    for i, xi in enumerate(xs):
        (newton_apply(cell, xi, base, h0=hs[i:i + 1]) * up[i:i + 1, :xi.shape[1]]).sum().backward()
    for a, b in zip(packed, [p.grad for p in cell.parameters()]):
        e = _rel(a.cpu(), b.cpu())
        print(f"  packed vs per-sequence param grad: {e:.2e}", flush=True)
        assert e <= 1e-5
    assert _rel(xp.grad[0, :150].cpu(), xs[0].grad[0].cpu()) <= 1e-5
    assert _rel(xp.grad[0, 150:].cpu(), xs[1].grad[0].cpu()) <= 1e-5
    assert _rel(hp.grad.cpu(), hs.grad.cpu()) <= 1e-5


def test_per_lane_walks_at_full_length_match_matrix_core_walks(monkeypatch):
    """At a size with more than a thousand chunk pairs the per-lane reverse
    walks take two chunks per wave (the other branch of their launch); their
    results against the matrix-core walks on the same inputs (fp32, the same
    arithmetic summed in a different order)."""
    from pararnn_amd import ops

    print("case full-length per-lane walks (two chunks per wave) vs matrix-core walks", flush=True)
    torch.manual_seed(5)
    B, T, H, din = 1, 32768, 8, 16
    d = 64 * H
    g = torch.Generator().manual_seed(6)
    p = GRUHeadParams(torch.randn(3 * d, din, generator=g) * 0.2,
                      torch.randn(3 * d, generator=g) * 0.1,
                      *(torch.randn(H, 64, 64, generator=g) * 0.1 for _ in range(3)))
    x = torch.randn(B, T, din, generator=g)
    wx = p.wx(x).to(DEV)
    states = torch.tanh(torch.randn(B, T, d, generator=g)).to(DEV)
    grad = torch.randn(B, T, d, generator=g).to(DEV)
    a = [t.to(DEV) for t in p.mats()]
    res = {}
    for walks in ("0", "1"):
        monkeypatch.setenv("PRNN_GRU_REV_MFMA", walks)
        res[walks] = ops.gru_head_backward_fused(wx, *a, None, states, grad)
    for i, k in enumerate(("g_wx", "g_a")):
        e = _rel(res["0"][i].cpu(), res["1"][i].cpu())
        print(f"  {k}: rel diff {e:.2e}", flush=True)
        assert e <= 1e-5, k
