"""GPU parity of the T=1 decode kernels (reference kernels/decode.py) against
the CPU oracle's cell step.  Every case prints its name before running."""

import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _slstm(d, dtype, seed, cap_hit=True):
    from pararnn_amd import ParaSLSTM

    torch.manual_seed(seed)
    cell = ParaSLSTM(16, d)
    with torch.no_grad():
        if cap_hit:
            cell.R.mul_(8.0)  # some entries beyond the 0.5 clamp
    return cell.to(DEV, dtype)


def _state(B, d, g, dtype):
    s = torch.randn(B, 4, d, generator=g)
    s[:, 1] = s[:, 1].abs() + 0.2  # normaliser n > 0
    return s.to(dtype)


def _ref_slstm(cell, state, wx):
    """Oracle step in fp32 on the widened inputs, rounded to the state dtype."""
    p = O.SLSTMParams(torch.zeros(4 * cell.d_h, 1), torch.zeros(4 * cell.d_h),
                      cell.R.detach().float().cpu(), eps=cell.eps, cap=cell.max_recurrent_norm)
    return O.slstm_step(p, state.float().cpu(), wx.float().cpu()).to(state.dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,d", [(1, 1), (3, 70), (8, 1024)])
def test_slstm_decode_matches_oracle(dtype, B, d):
    from pararnn_amd import decode_step

    print(f"case slstm decode B={B} d={d} {dtype}", flush=True)
    g = torch.Generator().manual_seed(B * 31 + d)
    cell = _slstm(d, dtype, 0)
    state = _state(B, d, g, dtype)
    wx = (torch.randn(B, 4 * d, generator=g) * 2).to(dtype)
    with torch.no_grad():
        out = decode_step(cell, state.to(DEV), wx=wx.to(DEV)).cpu()
    ref = _ref_slstm(cell, state, wx)
    if dtype == torch.float32:
        assert torch.allclose(out, ref, rtol=2e-6, atol=2e-6)
    else:  # same fp32 algebra, one rounding: at most one ulp of the dtype apart
        diff = (out.float() - ref.float()).abs()
        fi = torch.finfo(dtype)
        ulp = ref.float().abs() * fi.eps + fi.smallest_normal * fi.eps
        assert bool((diff <= ulp).all()), diff.max()


def test_slstm_decode_block_table_in_place_and_out():
    from pararnn_amd import decode_step

    print("case slstm decode block_table / out=", flush=True)
    g = torch.Generator().manual_seed(9)
    d = 96
    cell = _slstm(d, torch.float32, 1)
    pool = _state(7, d, g, torch.float32).to(DEV)
    before = pool.clone()
    bt = torch.tensor([5, 0, 3], dtype=torch.int64)
    wx = torch.randn(3, 4 * d, generator=g).to(DEV)
    with torch.no_grad():
        ret = decode_step(cell, pool, wx=wx, block_table=bt)
    assert ret.data_ptr() == pool.data_ptr()
    ref = _ref_slstm(cell, before[bt].cpu(), wx.cpu())
    assert torch.allclose(pool[bt].cpu(), ref, rtol=2e-6, atol=2e-6)
    untouched = [i for i in range(7) if i not in bt.tolist()]
    assert torch.equal(pool[untouched], before[untouched])
    # out= reuse without a block table
    state = _state(2, d, g, torch.float32).to(DEV)
    out = torch.full_like(state, float("nan"))
    with torch.no_grad():
        ret = decode_step(cell, state, wx=wx[:2], out=out)
    assert ret.data_ptr() == out.data_ptr()
    assert torch.allclose(out.cpu(), _ref_slstm(cell, state.cpu(), wx[:2].cpu()),
                          rtol=2e-6, atol=2e-6)


def test_slstm_decode_from_x_and_sequential_t1():
    from pararnn_amd import decode_step, sequential_apply

    print("case slstm decode from x, sequential_apply T=1", flush=True)
    g = torch.Generator().manual_seed(4)
    d = 64
    cell = _slstm(d, torch.float32, 2, cap_hit=False)
    state = _state(4, d, g, torch.float32).to(DEV)
    x = torch.randn(4, 1, 16, generator=g).to(DEV)
    with torch.no_grad():
        a = decode_step(cell, state, x)
        b = sequential_apply(cell, x, h0=state)[:, 0]
        c = cell.step(state, x[:, 0])
    assert torch.allclose(a, c, rtol=2e-6, atol=2e-6)
    assert torch.allclose(a, b, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("mix", ["diag", "head"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_gru_decode_matches_float64(mix, dtype):
    from pararnn_amd import ParaGRU, decode_step

    print(f"case gru decode {mix} {dtype}", flush=True)
    torch.manual_seed(3)
    g = torch.Generator().manual_seed(3)
    B, d = 5, 128
    cell = ParaGRU(8, d, mix=mix, n_heads=2 if mix == "head" else None).to(DEV, dtype)
    h = (torch.randn(B, d, generator=g) * 0.6).to(dtype)
    wx = torch.randn(B, 3 * d, generator=g).to(dtype)
    with torch.no_grad():
        out = decode_step(cell, h.to(DEV), wx=wx.to(DEV)).float().cpu()
    # float64 restatement of the step on the same (widened) inputs
    h64, wx64 = h.double(), wx.double()
    zx, rx, nx = wx64.chunk(3, dim=-1)
    if mix == "diag":
        az, ar, an = (t.detach().double().cpu() for t in cell.clipped_a())
        z = torch.sigmoid(az * h64 + zx)
        r = torch.sigmoid(ar * h64 + rx)
        n = torch.tanh(an * (h64 * r) + nx)
    else:
        A = [t.detach().double().cpu() for t in cell.clipped_a_head()]
        hv = h64.reshape(B, 2, 64)

        def mixv(v, a):
            return torch.matmul(v.unsqueeze(-2), a).squeeze(-2).reshape(B, d)

        z = torch.sigmoid(mixv(hv, A[0]) + zx)
        r = torch.sigmoid(mixv(hv, A[1]) + rx)
        n = torch.tanh(mixv(hv * r.reshape(B, 2, 64), A[2]) + nx)
    ref = (1 - z) * h64 + z * n
    tol = {torch.float32: 2e-6, torch.bfloat16: 2 ** -8, torch.float16: 2 ** -11}[dtype]
    err = ((out.double() - ref).abs() / (1 + ref.abs())).max().item()
    print(f"  rel err {err:.2e}", flush=True)
    assert err <= tol


def test_decode_graph_replay():
    from pararnn_amd import decode_step

    print("case slstm decode under hipGraph capture, 4 replays", flush=True)
    g = torch.Generator().manual_seed(12)
    d = 256
    cell = _slstm(d, torch.bfloat16, 5)
    state = _state(4, d, g, torch.bfloat16).to(DEV)
    wx = (torch.randn(4, 4 * d, generator=g)).to(torch.bfloat16).to(DEV)
    out = torch.empty_like(state)
    with torch.no_grad():
        eager = decode_step(cell, state, wx=wx).clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            decode_step(cell, state, wx=wx, out=out)  # warm up outside capture
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            decode_step(cell, state, wx=wx, out=out)
        for _ in range(4):
            out.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
