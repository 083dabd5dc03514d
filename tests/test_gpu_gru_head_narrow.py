"""ParaGRU(mix='head') with heads narrower than 64 channels: several heads share
one 64-channel kernel block as a block-diagonal 64 x 64 matrix (copy-free when
64 % d_head == 0 and the heads fill whole blocks, zero-padded otherwise).
Forward (fp32 and bf16), eq. 2.6 backward and T=1 decode against the CPU
oracle, whose head cell is written for any d_head.  Every case prints its name
before running."""

import pytest
import torch

import oracle as O
from oracle.backward import gru_head_backward

pytestmark = pytest.mark.gpu

DEV = "cuda:0"

# (n_heads, d_head): copy-free merges, a partly filled last block, and widths
# that do not divide 64
SHAPES = [(4, 32), (8, 16), (16, 4), (3, 32), (2, 48), (5, 20), (1, 1)]


def _cfg(K):
    from pararnn_amd import NewtonConfig

    return NewtonConfig(max_iters=K, residual_atol=None, residual_fail=None)


def _make(H, dh, seed, din=12):
    from pararnn_amd import ParaGRU

    torch.manual_seed(seed)
    cell = ParaGRU(din, H * dh, mix="head", n_heads=H)
    p = O.GRUHeadParams(cell.W_x.weight.detach().clone(), cell.W_x.bias.detach().clone(),
                        cell.A_z.detach().clone(), cell.A_r.detach().clone(),
                        cell.A_n.detach().clone())
    return cell, p


@pytest.mark.parametrize("H,dh", SHAPES)
def test_forward_fp32_vs_oracle(H, dh):
    from pararnn_amd import newton_apply

    print(f"case narrow heads forward fp32 H={H} d_head={dh}", flush=True)
    cell, p = _make(H, dh, 100 * H + dh)
    g = torch.Generator().manual_seed(H + dh)
    x = torch.randn(2, 333, 12, generator=g) * 1.5
    h0 = torch.randn(2, H * dh, generator=g) * 0.5
    with torch.no_grad():
        ref = O.gru_head_newton(p, x, max_iters=3, h0=h0)
        out = newton_apply(cell.to(DEV), x.to(DEV), _cfg(3), h0=h0.to(DEV)).cpu()
    err = (out - ref).abs().max().item()
    print(f"  max|gpu - oracle| {err:.2e}", flush=True)
    assert err <= 1e-5


@pytest.mark.parametrize("H,dh", [(4, 32), (2, 48)])
def test_forward_bf16_vs_oracle(H, dh):
    """bf16 storage: fp32 work inside the op, one rounding of the result, so
    the bar is against the oracle's fp32 algebra on the same bf16 operands."""
    from pararnn_amd import newton_apply

    print(f"case narrow heads forward bf16 H={H} d_head={dh}", flush=True)
    cell, _ = _make(H, dh, 7 * H + dh)
    cell = cell.to(torch.bfloat16)
    g = torch.Generator().manual_seed(3 * H + dh)
    x = torch.randn(2, 400, 12, generator=g).to(torch.bfloat16)
    p32 = O.GRUHeadParams(*(t.detach().float() for t in (cell.W_x.weight, cell.W_x.bias,
                                                          cell.A_z, cell.A_r, cell.A_n)))
    with torch.no_grad():
        wx = cell.W_x(x)  # the bf16 projection the op sees
        ref = O.gru_head_newton(p32, None, max_iters=3, wx=wx.float())
        out = newton_apply(cell.to(DEV), x.to(DEV), _cfg(3)).float().cpu()
    rel = ((out - ref).norm() / ref.norm()).item()
    print(f"  norm-rel vs fp32 algebra on bf16 operands {rel:.2e}", flush=True)
    assert rel <= 1e-2


@pytest.mark.parametrize("H,dh", [(4, 32), (3, 32), (5, 20)])
def test_backward_vs_float64(H, dh):
    from pararnn_amd import ops

    print(f"case narrow heads backward op H={H} d_head={dh}", flush=True)
    g = torch.Generator().manual_seed(H * 31 + dh)
    d, din, B, T = H * dh, 10, 2, 257
    p = O.GRUHeadParams(torch.randn(3 * d, din, generator=g) * 0.2,
                        torch.randn(3 * d, generator=g) * 0.1,
                        *(torch.randn(H, dh, dh, generator=g) * 0.2 for _ in range(3)))
    x = torch.randn(B, T, din, generator=g)
    h0 = torch.randn(B, d, generator=g) * 0.5
    states = torch.tanh(torch.randn(B, T, d, generator=g))
    grad = torch.randn(B, T, d, generator=g)
    wx = p.wx(x)
    g_wx, g_a, g_h0 = ops.gru_head_backward_fused(
        wx.to(DEV), *(a.to(DEV) for a in p.mats()), h0.to(DEV), states.to(DEV), grad.to(DEV))
    assert g_a.shape == (3, H, dh, dh)
    p64 = O.GRUHeadParams(*(v.double() for v in (p.W, p.b, p.A_z, p.A_r, p.A_n)))
    ref = gru_head_backward(p64, x.double(), states.double(), grad.double(), h0=h0.double(),
                            work=torch.float64, wx=wx.double())

    def rel(a, b):
        return ((a.cpu().double() - b).abs().max() / b.abs().max()).item()

    errs = {"g_wx": rel(g_wx, ref["g_wx"]), "h0": rel(g_h0, ref["h0"])}
    for i, k in enumerate(("A_z", "A_r", "A_n")):
        errs[k] = rel(g_a[i], ref[k])
    print("  rel err " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v <= 2e-5, k


@pytest.mark.parametrize("H,dh", [(4, 32), (8, 8)])
def test_decode_step_vs_oracle(H, dh):
    from pararnn_amd import can_decode_step, decode_step

    print(f"case narrow heads decode H={H} d_head={dh}", flush=True)
    cell, p = _make(H, dh, 5 * H + dh)
    cell = cell.to(DEV)
    g = torch.Generator().manual_seed(dh)
    h = torch.randn(6, H * dh, generator=g) * 0.5
    wx = torch.randn(6, 3 * H * dh, generator=g)
    assert can_decode_step(cell, h.to(DEV))
    with torch.no_grad():
        out = decode_step(cell, h.to(DEV), wx=wx.to(DEV)).cpu()
    ref = O.gru_head_step(p, h, wx)
    err = (out - ref).abs().max().item()
    print(f"  max|gpu - oracle| {err:.2e}", flush=True)
    assert err <= 2e-6
