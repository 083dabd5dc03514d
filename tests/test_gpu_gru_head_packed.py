"""Packed streams inside the head-GRU kernels: one stream (1, N, 3d) of S
sequences, the carry cut at every head (the chunk transfer of a chunk holding a
head is zero, each replay column restarts at a head from the sequence's h0
row), the eq. 2.6 backward resetting nu at each head and writing that
sequence's dL/dh0.  Checked against the oracle's per-sequence solves
(reference semantics: layout.py:93-138, solvers/scan.py:206-216) and the
rectangular kernels run on each sequence alone, with both replay and reverse
walk kernels.  Every case prints its name before running."""

import pytest
import torch

import oracle as O
from oracle.backward import gru_head_backward
from oracle.ragged import gru_head_newton_ragged

pytestmark = pytest.mark.gpu

DEV = "cuda:0"

# heads inside chunks and on chunk boundaries (chunks of 32 steps), single
# steps, a long sequence among short ones
LENGTHS = {
    "mixed": [1, 5, 37, 300, 2, 1, 64, 1000, 3, 129],
    "boundaries": [32, 31, 33, 64, 1, 95, 32],
    "tiny": [1] * 9 + [2] * 6 + [3] * 5,
    "one": [777],
    "long_short": [4100] + [17] * 30,
}


@pytest.fixture(params=["vec", "mfma"])
def walks(request, monkeypatch):
    """Run with each replay / reverse-walk kernel (per-lane mat-vecs or matrix
    cores)."""
    v = "1" if request.param == "mfma" else "0"
    monkeypatch.setenv("PRNN_GRU_REPLAY_MFMA", v)
    monkeypatch.setenv("PRNN_GRU_REV_MFMA", v)
    return request.param


def _params(H, dh, din, seed):
    g = torch.Generator().manual_seed(seed)
    d = H * dh
    return O.GRUHeadParams(torch.randn(3 * d, din, generator=g) * 0.3,
                           torch.randn(3 * d, generator=g) * 0.1,
                           *(torch.randn(H, dh, dh, generator=g) * 0.2 for _ in range(3)))


def _stream(lengths, d, din, seed, with_h0=True):
    g = torch.Generator().manual_seed(seed)
    n = sum(lengths)
    x = torch.randn(1, n, din, generator=g)
    h0 = torch.randn(len(lengths), d, generator=g) * 0.5 if with_h0 else None
    cs = torch.tensor([0] + lengths).cumsum(0)
    return x, h0, cs


@pytest.mark.parametrize("case", list(LENGTHS))
@pytest.mark.parametrize("K", [1, 3])
def test_packed_forward_fp32_vs_per_sequence_oracle(case, K, walks):
    from pararnn_amd import ops

    lengths = LENGTHS[case]
    print(f"case gru head packed fp32 {case} (S={len(lengths)}, N={sum(lengths)}) K={K} "
          f"walks={walks}", flush=True)
    H, dh, din = 2, 64, 12
    p = _params(H, dh, din, 17 + K)
    x, h0, cs = _stream(lengths, H * dh, din, 3 + K, with_h0=case != "tiny")
    wx = p.wx(x)
    with torch.no_grad():
        out = ops.newton_gru_head_fused(wx.to(DEV), *(a.to(DEV) for a in p.mats()),
                                        None if h0 is None else h0.to(DEV), cs.to(DEV),
                                        max_iters=K, omega=1.0).cpu()
    ref = gru_head_newton_ragged(p, x, cs, max_iters=K, h0=h0)
    err = (out - ref).abs().max().item()
    print(f"  max|gpu - per-sequence oracle| {err:.2e}", flush=True)
    assert err <= 1e-5


@pytest.mark.parametrize("case", ["mixed", "boundaries", "long_short"])
def test_packed_backward_fp32_vs_per_sequence_float64(case, walks):
    """The eq. 2.6 op on a packed stream at a given H*: dL/dwx, dL/dA (summed
    over the sequences) and each sequence's dL/dh0 against the float64 oracle
    run on each sequence alone."""
    from pararnn_amd import ops

    lengths = LENGTHS[case]
    print(f"case gru head packed backward fp32 {case} walks={walks}", flush=True)
    H, dh, din = 2, 64, 10
    d = H * dh
    p = _params(H, dh, din, 40)
    x, h0, cs = _stream(lengths, d, din, 41)
    g = torch.Generator().manual_seed(42)
    n = sum(lengths)
    states = torch.tanh(torch.randn(1, n, d, generator=g))
    grad = torch.randn(1, n, d, generator=g)
    wx = p.wx(x)
    g_wx, g_a, g_h0 = ops.gru_head_backward_fused(
        wx.to(DEV), *(a.to(DEV) for a in p.mats()), h0.to(DEV), states.to(DEV), grad.to(DEV),
        cs.to(DEV))
    assert g_h0.shape == (len(lengths), d)
    p64 = O.GRUHeadParams(*(v.double() for v in (p.W, p.b, p.A_z, p.A_r, p.A_n)))
    ex_wx, ex_a, ex_h0 = [], [0.0, 0.0, 0.0], []
    for s, (a, b) in enumerate(zip(cs[:-1].tolist(), cs[1:].tolist())):
        r = gru_head_backward(p64, x[:, a:b].double(), states[:, a:b].double(),
                              grad[:, a:b].double(), h0=h0[s:s + 1].double(),
                              work=torch.float64, wx=wx[:, a:b].double())
        ex_wx.append(r["g_wx"])
        ex_h0.append(r["h0"])
        for i, k in enumerate(("A_z", "A_r", "A_n")):
            ex_a[i] = ex_a[i] + r[k]
    ex_wx, ex_h0 = torch.cat(ex_wx, 1), torch.cat(ex_h0, 0)

    def rel(a, b):
        return ((a.cpu().double() - b).abs().max() / b.abs().max()).item()

    errs = {"g_wx": rel(g_wx, ex_wx), "h0": rel(g_h0, ex_h0)}
    for i, k in enumerate(("A_z", "A_r", "A_n")):
        errs[k] = rel(g_a[i], ex_a[i])
    print("  rel err " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v <= 2e-5, k


def test_packed_bf16_vs_each_sequence_alone():
    """bf16 storage: the packed stream against the rectangular kernels on each
    sequence alone (same algorithm; only the chunk boundaries differ)."""
    from pararnn_amd import ops

    lengths = LENGTHS["mixed"]
    print("case gru head packed bf16 vs per-sequence rectangular launches", flush=True)
    H, dh, din = 4, 64, 16
    p = _params(H, dh, din, 50)
    x, h0, cs = _stream(lengths, H * dh, din, 51)
    wx = p.wx(x).to(DEV, torch.bfloat16)
    mats = [a.to(DEV, torch.bfloat16) for a in p.mats()]
    hd = h0.to(DEV, torch.bfloat16)
    with torch.no_grad():
        out = ops.newton_gru_head_fused(wx, *mats, hd, cs.to(DEV), max_iters=3,
                                        omega=1.0).float()
        parts = [ops.newton_gru_head_fused(wx[:, a:b].contiguous(), *mats, hd[s:s + 1],
                                           max_iters=3, omega=1.0).float()
                 for s, (a, b) in enumerate(zip(cs[:-1].tolist(), cs[1:].tolist()))]
    ref = torch.cat(parts, 1)
    rel = ((out - ref).norm() / ref.norm()).item()
    print(f"  norm-rel {rel:.2e}", flush=True)
    assert rel <= 1e-2


@pytest.mark.parametrize("H,dh", [(4, 32), (3, 20)])
def test_packed_narrow_heads(H, dh):
    """Heads narrower than 64 channels (block-diagonal kernel blocks) on a
    packed stream."""
    from pararnn_amd import ops

    lengths = LENGTHS["boundaries"]
    print(f"case gru head packed narrow heads H={H} d_head={dh}", flush=True)
    p = _params(H, dh, 9, 60 + dh)
    x, h0, cs = _stream(lengths, H * dh, 9, 61)
    wx = p.wx(x)
    with torch.no_grad():
        out = ops.newton_gru_head_fused(wx.to(DEV), *(a.to(DEV) for a in p.mats()),
                                        h0.to(DEV), cs.to(DEV), max_iters=3, omega=1.0).cpu()
    ref = gru_head_newton_ragged(p, x, cs, max_iters=3, h0=h0)
    err = (out - ref).abs().max().item()
    print(f"  max|gpu - per-sequence oracle| {err:.2e}", flush=True)
    assert err <= 1e-5


def test_packed_newton_apply_block_table_and_grad():
    """newton_apply on a packed head-GRU stream: a paged h0 (block_table rows
    of a pool) equals the gathered dense h0 bit for bit, and the gradients
    through the packed solve equal the per-sequence solves' sum."""
    from pararnn_amd import NewtonConfig, ParaGRU, newton_apply

    print("case gru head packed newton_apply block_table and gradients", flush=True)
    torch.manual_seed(70)
    cell = ParaGRU(8, 128, mix="head", n_heads=2).to(DEV)
    lengths = [40, 1, 77, 33]
    g = torch.Generator().manual_seed(71)
    n = sum(lengths)
    x = torch.randn(1, n, 8, generator=g).to(DEV)
    pool = (torch.randn(9, 128, generator=g) * 0.5).to(DEV)
    bt = torch.tensor([8, 0, 3, 3], device=DEV)
    cs = torch.tensor([0] + lengths).cumsum(0).to(DEV)
    cfg = NewtonConfig(max_iters=3, residual_atol=None, residual_fail=None)
    with torch.no_grad():
        a = newton_apply(cell, x, cfg, h0=pool, cu_seqlens=cs, block_table=bt)
        b = newton_apply(cell, x, cfg, h0=pool[bt], cu_seqlens=cs)
    assert torch.equal(a, b)
    up = torch.randn(1, n, 128, generator=g).to(DEV)
    h0 = pool[bt].clone()
    xa, ha = x.clone().requires_grad_(True), h0.clone().requires_grad_(True)
    (newton_apply(cell, xa, cfg, h0=ha, cu_seqlens=cs) * up).sum().backward()
    ga = {k: v.grad.clone() for k, v in cell.named_parameters()}
    cell.zero_grad()
    xb, hb = x.clone().requires_grad_(True), h0.clone().requires_grad_(True)
    off = 0
    for s, m in enumerate(lengths):
        (newton_apply(cell, xb[:, off:off + m], cfg, h0=hb[s:s + 1]) *
         up[:, off:off + m]).sum().backward()
        off += m
    for k, v in cell.named_parameters():
        e = ((ga[k] - v.grad).abs().max() / v.grad.abs().max()).item()
        print(f"  grad {k}: rel diff {e:.2e}", flush=True)
        assert e <= 1e-5
    for k, u, w in (("x", xa.grad, xb.grad), ("h0", ha.grad, hb.grad)):
        e = ((u - w).abs().max() / w.abs().max()).item()
        print(f"  grad {k}: rel diff {e:.2e}", flush=True)
        assert e <= 1e-5


def test_packed_fp16_vs_each_sequence_alone():
    """fp16 storage: the packed stream against the rectangular kernels on each
    sequence alone."""
    from pararnn_amd import ops

    lengths = LENGTHS["mixed"]
    print("case gru head packed fp16 vs per-sequence rectangular launches", flush=True)
    H, dh, din = 4, 64, 16
    p = _params(H, dh, din, 80)
    x, h0, cs = _stream(lengths, H * dh, din, 81)
    wx = p.wx(x).to(DEV, torch.float16)
    mats = [a.to(DEV, torch.float16) for a in p.mats()]
    hd = h0.to(DEV, torch.float16)
    with torch.no_grad():
        out = ops.newton_gru_head_fused(wx, *mats, hd, cs.to(DEV), max_iters=3, omega=1.0)
        parts = [ops.newton_gru_head_fused(wx[:, a:b].contiguous(), *mats, hd[s:s + 1],
                                           max_iters=3, omega=1.0)
                 for s, (a, b) in enumerate(zip(cs[:-1].tolist(), cs[1:].tolist()))]
    assert out.dtype == torch.float16
    ref = torch.cat(parts, 1).float()
    rel = ((out.float() - ref).norm() / ref.norm()).item()
    print(f"  norm-rel {rel:.2e}", flush=True)
    assert rel <= 2e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_packed_backward_narrow_vs_each_sequence_alone(dtype, walks):
    """16-bit storage: the eq. 2.6 backward on a packed stream against the
    rectangular backward on each sequence alone: dL/dwx, each sequence's
    dL/dh0 row, and dL/dA summed over the sequences."""
    from pararnn_amd import ops

    lengths = LENGTHS["mixed"]
    print(f"case gru head packed backward {dtype} walks={walks}", flush=True)
    H, dh, din = 2, 64, 10
    d = H * dh
    p = _params(H, dh, din, 90)
    x, h0, cs = _stream(lengths, d, din, 91)
    g = torch.Generator().manual_seed(92)
    n = sum(lengths)
    states = torch.tanh(torch.randn(1, n, d, generator=g)).to(DEV, dtype)
    grad = torch.randn(1, n, d, generator=g).to(DEV, dtype)
    wx = p.wx(x).to(DEV, dtype)
    mats = [a.to(DEV, dtype) for a in p.mats()]
    hd = h0.to(DEV, dtype)
    g_wx, g_a, g_h0 = ops.gru_head_backward_fused(wx, *mats, hd, states, grad, cs.to(DEV))
    e_wx, e_h0, e_a = [], [], torch.zeros_like(g_a)
    for s, (a, b) in enumerate(zip(cs[:-1].tolist(), cs[1:].tolist())):
        q_wx, q_a, q_h0 = ops.gru_head_backward_fused(
            wx[:, a:b].contiguous(), *mats, hd[s:s + 1], states[:, a:b].contiguous(),
            grad[:, a:b].contiguous())
        e_wx.append(q_wx)
        e_h0.append(q_h0)
        e_a += q_a
    e_wx, e_h0 = torch.cat(e_wx, 1), torch.cat(e_h0, 0)

    def nrel(u, v):
        u, v = u.double(), v.double()
        return ((u - v).norm() / v.norm()).item()

    errs = {"g_wx": nrel(g_wx, e_wx), "g_h0": nrel(g_h0, e_h0), "g_a": nrel(g_a, e_a)}
    print("  norm-rel " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    assert g_wx.dtype == dtype
    assert errs["g_wx"] <= (4e-3 if dtype == torch.bfloat16 else 1e-3)
    # g_h0 is fp32 from the walk's carries; g_A is contracted from the stored
    # (16-bit) gate gradients, so a one-ulp move there shows up in it too
    assert errs["g_h0"] <= 1e-4 and errs["g_a"] <= 2e-3
