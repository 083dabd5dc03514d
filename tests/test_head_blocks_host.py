"""Narrow heads on 64-channel blocks (pararnn_amd.head_blocks), on the CPU: the
channel and weight maps are inverse to each other, and the head-GRU Newton
solve of the block layout (oracle, float64) equals the narrow cell's own
solve, padded channels staying at zero."""

import pytest
import torch

import oracle as O
from pararnn_amd.head_blocks import HeadBlocks

SHAPES = [(4, 32), (8, 16), (3, 32), (2, 48), (5, 20), (1, 1), (2, 64)]


@pytest.mark.parametrize("H,dh", SHAPES)
def test_maps_round_trip(H, dh):
    hb = HeadBlocks(H, dh, torch.device("cpu"))
    a = torch.randn(H, dh, dh)
    m = hb.matrices(a)
    assert m.shape == (hb.n_blocks, 64, 64)
    assert torch.equal(hb.head_grads(m.unsqueeze(0))[0], a)
    # everything off the heads' diagonal blocks is zero
    assert m.abs().sum().item() == pytest.approx(a.abs().sum().item(), rel=1e-6)
    x = torch.randn(2, 5, 3 * H * dh)
    xb = hb.to_blocks(x, 3)
    assert xb.shape[-1] == 3 * hb.d_pad
    assert torch.equal(hb.from_blocks(xb, 3), x)
    assert hb.identity == (64 % dh == 0 and H % (64 // dh) == 0)


@pytest.mark.parametrize("H,dh", [(3, 32), (2, 48), (5, 20), (4, 16)])
def test_block_layout_solve_equals_narrow_solve(H, dh):
    g = torch.Generator().manual_seed(H * 100 + dh)
    d, din = H * dh, 7
    p = O.GRUHeadParams(torch.randn(3 * d, din, generator=g, dtype=torch.float64) * 0.3,
                        torch.randn(3 * d, generator=g, dtype=torch.float64) * 0.1,
                        *(torch.randn(H, dh, dh, generator=g, dtype=torch.float64) * 0.3
                          for _ in range(3)))
    x = torch.randn(2, 40, din, generator=g, dtype=torch.float64)
    h0 = torch.randn(2, d, generator=g, dtype=torch.float64) * 0.5
    wx = p.wx(x)
    want = O.gru_head_newton(p, None, max_iters=4, h0=h0, wx=wx)
    hb = HeadBlocks(H, dh, torch.device("cpu"))
    pb = O.GRUHeadParams(p.W, p.b, *(hb.matrices(a) for a in (p.A_z, p.A_r, p.A_n)))
    out = O.gru_head_newton(pb, None, max_iters=4, h0=hb.to_blocks(h0), wx=hb.to_blocks(wx, 3))
    assert torch.allclose(hb.from_blocks(out), want, rtol=0, atol=1e-12)
    if not hb.identity:
        pad = torch.ones(hb.d_pad, dtype=torch.bool)
        pad[hb.chan] = False
        assert out[..., pad].abs().max().item() == 0.0


def test_wider_than_a_block_is_rejected():
    with pytest.raises(TypeError, match="d_head <= 64"):
        HeadBlocks(2, 128, torch.device("cpu"))
