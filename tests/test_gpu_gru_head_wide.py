"""ParaGRU(mix='head') with wide heads, 64 < d_head <= 128 (the tier of the
reference's streamed head kernel, kernels/newton_gru_head.py:121-150): the
gates at the iterate as GEMMs, the Newton solve and the eq. 2.6 adjoint as HIP
walks per (sequence, head).  Forward (fp32, bf16; rectangular and packed) and
backward against the CPU oracle, whose head cell is written for any d_head.
Every case prints its name before running."""

import pytest
import torch

import oracle as O
from oracle.backward import gru_head_backward

pytestmark = pytest.mark.gpu

DEV = "cuda:0"

SHAPES = [(2, 96), (1, 128), (3, 80), (2, 65)]


def _cfg(K, **kw):
    from pararnn_amd import NewtonConfig

    return NewtonConfig(max_iters=K, residual_atol=None, residual_fail=None, **kw)


def _make(H, dh, seed, din=12):
    from pararnn_amd import ParaGRU

    torch.manual_seed(seed)
    cell = ParaGRU(din, H * dh, mix="head", n_heads=H)
    p = O.GRUHeadParams(cell.W_x.weight.detach().clone(), cell.W_x.bias.detach().clone(),
                        cell.A_z.detach().clone(), cell.A_r.detach().clone(),
                        cell.A_n.detach().clone())
    return cell, p


@pytest.mark.parametrize("H,dh", SHAPES)
@pytest.mark.parametrize("K", [0, 1, 3])
def test_forward_fp32_vs_oracle(H, dh, K):
    from pararnn_amd import newton_apply

    print(f"case wide heads forward fp32 H={H} d_head={dh} K={K}", flush=True)
    cell, p = _make(H, dh, 100 * H + dh)
    g = torch.Generator().manual_seed(H + dh)
    x = torch.randn(2, 333, 12, generator=g) * 1.5
    h0 = torch.randn(2, H * dh, generator=g) * 0.5
    with torch.no_grad():
        ref = O.gru_head_newton(p, x, max_iters=K, h0=h0)
        out = newton_apply(cell.to(DEV), x.to(DEV), _cfg(K), h0=h0.to(DEV)).cpu()
    err = (out - ref).abs().max().item()
    print(f"  max|gpu - oracle| {err:.2e}", flush=True)
    assert err <= 1e-5


def test_forward_converges_to_sequential():
    """Enough Newton iterations land on the sequential unroll (the fixed point)."""
    from pararnn_amd import newton_apply, sequential_apply

    print("case wide heads K=8 vs sequential unroll", flush=True)
    cell, _ = _make(2, 128, 5)
    cell = cell.to(DEV)
    x = torch.randn(3, 500, 12, device=DEV)
    with torch.no_grad():
        par = newton_apply(cell, x, _cfg(8))
        seq = sequential_apply(cell, x)
    err = (par - seq).abs().max().item()
    print(f"  max|newton - sequential| {err:.2e}", flush=True)
    assert err <= 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("H,dh", [(2, 96), (1, 128)])
def test_forward_bf16_vs_oracle(H, dh, dtype):
    """16-bit storage: fp32 work on the 16-bit operands, one rounding of the
    result.  Bar (relative): 2^-8 for bf16, 2^-9 for fp16 -- the result's
    rounding plus that of wx, whose GEMM runs on the CPU for the oracle."""
    from pararnn_amd import newton_apply

    print(f"case wide heads forward {dtype} H={H} d_head={dh}", flush=True)
    cell, _ = _make(H, dh, 7 * H + dh)
    cell = cell.to(dtype)
    g = torch.Generator().manual_seed(3 * H + dh)
    x = torch.randn(2, 400, 12, generator=g).to(dtype)
    p32 = O.GRUHeadParams(*(t.detach().float() for t in (cell.W_x.weight, cell.W_x.bias,
                                                          cell.A_z, cell.A_r, cell.A_n)))
    with torch.no_grad():
        wx = cell.W_x(x)
        ref = O.gru_head_newton(p32, None, max_iters=3, wx=wx.float())
        out = newton_apply(cell.to(DEV), x.to(DEV), _cfg(3)).float().cpu()
    rel = ((out - ref).abs().max() / ref.abs().max()).item()
    print(f"  max-rel vs fp32 algebra on 16-bit operands {rel:.2e}", flush=True)
    assert rel <= (2 ** -8 if dtype == torch.bfloat16 else 2 ** -9)


@pytest.mark.parametrize("H,dh", [(2, 96), (1, 128), (3, 72)])
@pytest.mark.parametrize("with_h0", [True, False])
def test_backward_vs_float64(H, dh, with_h0):
    from pararnn_amd import ops

    print(f"case wide heads backward op H={H} d_head={dh} h0={with_h0}", flush=True)
    g = torch.Generator().manual_seed(H * 31 + dh)
    d, din, B, T = H * dh, 10, 2, 257
    p = O.GRUHeadParams(torch.randn(3 * d, din, generator=g) * 0.2,
                        torch.randn(3 * d, generator=g) * 0.1,
                        *(torch.randn(H, dh, dh, generator=g) * 0.1 for _ in range(3)))
    x = torch.randn(B, T, din, generator=g)
    h0 = torch.randn(B, d, generator=g) * 0.5 if with_h0 else None
    states = torch.tanh(torch.randn(B, T, d, generator=g))
    grad = torch.randn(B, T, d, generator=g)
    wx = p.wx(x)
    g_wx, g_a, g_h0 = ops.gru_head_backward_fused(
        wx.to(DEV), *(a.to(DEV) for a in p.mats()), None if h0 is None else h0.to(DEV),
        states.to(DEV), grad.to(DEV))
    assert g_a.shape == (3, H, dh, dh) and g_wx.shape == wx.shape
    p64 = O.GRUHeadParams(*(v.double() for v in (p.W, p.b, p.A_z, p.A_r, p.A_n)))
    ref = gru_head_backward(p64, x.double(), states.double(), grad.double(),
                            h0=None if h0 is None else h0.double(), work=torch.float64,
                            wx=wx.double())

    def rel(a, b):
        return ((a.cpu().double() - b).abs().max() / b.abs().max()).item()

    errs = {"g_wx": rel(g_wx, ref["g_wx"])}
    if with_h0:
        errs["h0"] = rel(g_h0, ref["h0"])
    for i, k in enumerate(("A_z", "A_r", "A_n")):
        errs[k] = rel(g_a[i], ref[k])
    print("  rel err " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v <= 2e-5, k


def test_autograd_end_to_end_vs_float64():
    """newton_apply + backward through the wide tier (clamp masks, W_x VJP),
    against float64 autograd through the sequential unroll at convergence."""
    from pararnn_amd import newton_apply

    print("case wide heads autograd d_head=128", flush=True)
    cell, p = _make(2, 128, 42, din=9)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 150, 9, generator=g)
    h0 = torch.randn(2, 256, generator=g) * 0.5
    up = torch.randn(2, 150, 256, generator=g)
    cell = cell.to(DEV)
    xg = x.to(DEV).requires_grad_(True)
    h0g = h0.to(DEV).requires_grad_(True)
    out = newton_apply(cell, xg, _cfg(8), h0=h0g)
    (out * up.to(DEV)).sum().backward()
    # float64 reference: autograd through the oracle's sequential unroll
    p64 = [t.detach().double().requires_grad_(True) for t in (p.W, p.b, p.A_z, p.A_r, p.A_n)]
    x64 = x.double().requires_grad_(True)
    h064 = h0.double().requires_grad_(True)
    q = O.GRUHeadParams(*p64)
    seq = O.gru_head_sequential(q, x64, h0=h064)
    (seq * up.double()).sum().backward()
    pairs = [("x", xg.grad, x64.grad), ("h0", h0g.grad, h064.grad),
             ("W_x", cell.W_x.weight.grad, p64[0].grad), ("A_z", cell.A_z.grad, p64[2].grad),
             ("A_r", cell.A_r.grad, p64[3].grad), ("A_n", cell.A_n.grad, p64[4].grad)]
    for name, got, want in pairs:
        rel = ((got.cpu().double() - want).abs().max() / want.abs().max()).item()
        print(f"  d{name} rel err vs float64 {rel:.2e}", flush=True)
        assert rel <= 1e-4, name


@pytest.mark.parametrize("paged", [False, True])
def test_packed_stream_vs_each_sequence_alone(paged):
    """cu_seqlens: one walk per (sequence, head) over its own steps from its
    own h0 row (a block_table row of a pool when paged); the backward's dL/dh0
    is per sequence."""
    from pararnn_amd import newton_apply

    print(f"case wide heads packed stream paged={paged}", flush=True)
    cell, p = _make(2, 96, 77)
    lengths = [130, 1, 64, 201]
    cs = torch.tensor([0] + lengths).cumsum(0)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, int(cs[-1]), 12, generator=g)
    h0 = torch.randn(len(lengths), 192, generator=g) * 0.5
    cell = cell.to(DEV)
    with torch.no_grad():
        if paged:
            pool = torch.randn(7, 192, generator=g)
            table = torch.tensor([3, 0, 6, 2], dtype=torch.int32)
            pool[table.long()] = h0
            out = newton_apply(cell, x.to(DEV), _cfg(3), h0=pool.to(DEV),
                               cu_seqlens=cs.to(DEV), block_table=table.to(DEV)).cpu()
        else:
            out = newton_apply(cell, x.to(DEV), _cfg(3), h0=h0.to(DEV),
                               cu_seqlens=cs.to(DEV)).cpu()
    worst = 0.0
    for s, (a, b) in enumerate(zip(cs[:-1].tolist(), cs[1:].tolist())):
        ref = O.gru_head_newton(p, x[:, a:b], max_iters=3, h0=h0[s:s + 1])
        worst = max(worst, (out[:, a:b] - ref).abs().max().item())
    print(f"  max|packed - each alone (oracle)| {worst:.2e}", flush=True)
    assert worst <= 1e-5
    if paged:
        return
    xg = x.to(DEV).requires_grad_(True)
    h0g = h0.to(DEV).requires_grad_(True)
    up = torch.randn(out.shape, generator=g)
    (newton_apply(cell, xg, _cfg(3), h0=h0g, cu_seqlens=cs.to(DEV)) * up.to(DEV)).sum().backward()
    gx = torch.zeros_like(x)
    gh = torch.zeros_like(h0)
    for s, (a, b) in enumerate(zip(cs[:-1].tolist(), cs[1:].tolist())):
        xs = x[:, a:b].to(DEV).requires_grad_(True)
        hs = h0[s:s + 1].to(DEV).requires_grad_(True)
        (newton_apply(cell, xs, _cfg(3), h0=hs) * up[:, a:b].to(DEV)).sum().backward()
        gx[:, a:b] = xs.grad.cpu()
        gh[s:s + 1] = hs.grad.cpu()
    ex = (xg.grad.cpu() - gx).abs().max().item() / gx.abs().max().item()
    eh = (h0g.grad.cpu() - gh).abs().max().item() / gh.abs().max().item()
    print(f"  packed vs per-sequence gradients: x {ex:.2e}, h0 {eh:.2e}", flush=True)
    assert ex <= 1e-5 and eh <= 1e-5


def test_wider_than_128_is_refused():
    from pararnn_amd import ParaGRU, newton_apply

    cell = ParaGRU(4, 136, mix="head", n_heads=1).to(DEV)
    with pytest.raises(TypeError, match="128"):
        with torch.no_grad():
            newton_apply(cell, torch.randn(1, 5, 4, device=DEV), _cfg(2))


def test_stacked_layers_and_verify_agreement():
    """A two-layer ParaRNN of wide heads: train() (Newton per layer) against
    eval() (sequential unroll per layer), and verify_agreement's verdict at
    its default tolerance."""
    from pararnn_amd import NewtonConfig, ParaGRU, ParaRNN, verify_agreement

    print("case wide heads ParaRNN 2 layers", flush=True)
    torch.manual_seed(3)
    cell = ParaGRU(16, 192, mix="head", n_heads=2)
    cfg = NewtonConfig(max_iters=6, residual_atol=None, residual_fail=None)
    model = ParaRNN(cell, num_layers=2, config=cfg).to(DEV)
    x = torch.randn(2, 300, 16, device=DEV)
    with torch.no_grad():
        model.train()
        y = model(x)
        model.eval()
        ys = model(x)
    err = (y - ys).abs().max().item()
    print(f"  max|train - eval| {err:.2e}", flush=True)
    assert err <= 1e-5
    rep = verify_agreement(cell.to(DEV), torch.randn(2, 300, 16, device=DEV),
                           config=NewtonConfig(max_iters=6))
    print(f"  verify_agreement max_abs {rep.max_abs:.2e} ok={rep.ok}", flush=True)
    assert rep.ok


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("K", [2, 5])
def test_one_launch_matches_launch_per_iteration(packed, K, monkeypatch):
    """K >= 2 runs all iterations in one launch (gate workgroups feeding the
    walks, iteration k a few blocks behind k - 1, gates and iterates passed
    as tagged words); PARARNN_AMD_WIDE_FUSED=0 runs the gates kernel and one
    walk per iteration.  The same arithmetic: they agree to float32 rounding,
    and no wait gives up (PARARNN_AMD_CHECK_STATUS=1)."""
    from pararnn_amd import newton_apply

    print(f"case wide heads one launch vs per iteration packed={packed} K={K}", flush=True)
    cell, _ = _make(2, 128, 11 + K)
    cell = cell.to(DEV)
    g = torch.Generator().manual_seed(K)
    if packed:
        lengths = [700, 3, 129, 1200, 17]
        cs = torch.tensor([0] + lengths).cumsum(0).to(DEV)
        x = torch.randn(1, int(cs[-1]), 12, generator=g).to(DEV)
        h0 = (torch.randn(len(lengths), 256, generator=g) * 0.5).to(DEV)
        kw = {"cu_seqlens": cs}
    else:
        x = torch.randn(3, 1500, 12, generator=g).to(DEV)
        h0 = (torch.randn(3, 256, generator=g) * 0.5).to(DEV)
        kw = {}
    monkeypatch.setenv("PARARNN_AMD_CHECK_STATUS", "1")
    with torch.no_grad():
        one = newton_apply(cell, x, _cfg(K), h0=h0, **kw)
        monkeypatch.setenv("PARARNN_AMD_WIDE_FUSED", "0")
        per = newton_apply(cell, x, _cfg(K), h0=h0, **kw)
    err = (one - per).abs().max().item()
    print(f"  max|one launch - per iteration| {err:.2e}", flush=True)
    assert torch.isfinite(one).all() and err <= 1e-5


def test_one_launch_more_workgroups_than_fit_at_once(monkeypatch):
    """K x B x H = 3 x 64 x 8 = 1536 (iteration, sequence, head) triples,
    a gate workgroup and a walk each: 3072 one-launch workgroups, more than
    the GPU holds at once.  The ticket order
    (iteration-major, gates before walks) lets every waiting workgroup find
    what it waits on running or done, so the solve completes without a wait
    giving up, equal to one launch per iteration."""
    from pararnn_amd import NewtonConfig, ParaGRU, newton_apply

    print("case wide heads one launch, 3072 workgroups (B=64, H=8, K=3)", flush=True)
    torch.manual_seed(21)
    cell = ParaGRU(16, 1024, mix="head", n_heads=8).to(DEV)
    x = torch.randn(64, 96, 16, device=DEV)
    cfg = NewtonConfig(max_iters=3, residual_atol=None, residual_fail=None)
    monkeypatch.setenv("PARARNN_AMD_CHECK_STATUS", "1")
    with torch.no_grad():
        one = newton_apply(cell, x, cfg)
        monkeypatch.setenv("PARARNN_AMD_WIDE_FUSED", "0")
        per = newton_apply(cell, x, cfg)
    err = (one - per).abs().max().item()
    print(f"  max|one launch - per iteration| {err:.2e}", flush=True)
    assert err <= 1e-5


def test_one_launch_workspace_cap_falls_back(monkeypatch):
    """A solve whose one-launch workspace exceeds the cap (here: any) runs one
    launch per iteration: the same result as PARARNN_AMD_WIDE_FUSED=0."""
    from pararnn_amd import newton_apply, ops

    print("case wide heads one-launch workspace cap", flush=True)
    cell, _ = _make(2, 96, 5)
    cell = cell.to(DEV)
    x = torch.randn(2, 300, 12, generator=torch.Generator().manual_seed(3)).to(DEV)
    with torch.no_grad():
        monkeypatch.setattr(ops, "_wide_workspace_cap", lambda dev: 0)
        capped = newton_apply(cell, x, _cfg(3))
        monkeypatch.setenv("PARARNN_AMD_WIDE_FUSED", "0")
        per = newton_apply(cell, x, _cfg(3))
    assert torch.isfinite(capped).all() and torch.equal(capped, per)


@pytest.mark.parametrize("dh", [96, 65, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gates_kernel_matches_the_oracle_cell(dtype, dh):
    """prnn_gru_wide_gates (fp32 matrix-core GEMMs) against the oracle's head
    cell (reference cells/para_gru.py:414-467) at the same previous states,
    with h0 rows at the sequence starts, d_head = 96 (whole 16-channel tiles
    dead), 65 (a tile with one live channel, a contraction block with one
    live entry) and 128, and a row count that is not a multiple of the
    16-row tile."""
    from oracle.gru_head import _acts
    from pararnn_amd import ops

    print(f"case wide heads gates kernel {dtype} d_head={dh}", flush=True)
    g = torch.Generator().manual_seed(dh)
    H, B, T = 2, 3, 37
    d = H * dh
    p = O.GRUHeadParams(torch.randn(3 * d, 5, generator=g), torch.randn(3 * d, generator=g),
                        *(torch.randn(H, dh, dh, generator=g) * 0.1 for _ in range(3)))
    wx = torch.randn(B, T, 3 * d, generator=g).to(dtype)
    states = torch.randn(B, T, d, generator=g)
    h0 = torch.randn(B, d, generator=g)
    mats = tuple(m.to(dtype) for m in p.mats())
    hp = ops._wide_prev(states, h0, None)
    code = {torch.float32: 0, torch.bfloat16: 1}[dtype]
    z, r, n = ops._wide_gates(wx.to(DEV), hp.to(DEV).contiguous(),
                              tuple(m.to(DEV).contiguous() for m in mats), code)
    # the oracle's cell in float64 on the same (fp32- or bf16-valued) operands;
    # bar: a few fp32 ulps of pre-activations up to ~4 in magnitude (sums of
    # up to 128 products) plus the device's fast sigmoid and tanh
    p64 = O.GRUHeadParams(p.W.double(), p.b.double(), *(m.double() for m in mats))
    a = _acts(p64, hp.double(), wx.double())
    for name, got, want in (("z", z, a["z"]), ("r", r, a["r"]), ("n", n, a["n"])):
        err = (got.cpu().double() - want.reshape(B, T, d)).abs().max().item()
        print(f"  {name}: max|gpu - float64 oracle| {err:.2e}", flush=True)
        assert err <= 2e-6
