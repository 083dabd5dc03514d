"""GPU parity of packed ragged batches (``cu_seqlens``) and paged ``h0``
(``block_table``) against the reference's golden vectors and the oracle.
Every case prints its name before running."""

import pytest
import torch
from conftest import load_golden

import oracle as O
from oracle.ragged import slstm_newton_ragged

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _cfg(K, P=None, **kw):
    from pararnn_amd import NewtonConfig

    return NewtonConfig(max_iters=K, picard_iters=P, residual_atol=None, residual_fail=None,
                        picard_adapt=False, **kw)


def _slstm_cell(t, m):
    from pararnn_amd import ParaSLSTM

    cell = ParaSLSTM(m["d_in"], m["d"])
    with torch.no_grad():
        cell.W_x.weight.copy_(t["W"])
        cell.W_x.bias.copy_(t["b"])
        cell.R.copy_(t["R"])
    return cell.to(DEV)


def test_slstm_ragged_matches_reference():
    from pararnn_amd import newton_apply, sequential_apply

    print("case slstm ragged fp32 (lengths 37, 100, 64; h0 per sequence)", flush=True)
    t, m = load_golden("slstm_ragged_fp32")
    cell = _slstm_cell(t, m)
    cs = t["cu_seqlens"]
    with torch.no_grad():
        H = newton_apply(cell, t["x"].to(DEV), _cfg(m["K"], m["P"]), h0=t["h0"].to(DEV),
                         cu_seqlens=cs.to(DEV)).cpu()
        Hs = sequential_apply(cell, t["x"].to(DEV), t["h0"].to(DEV), cu_seqlens=cs).cpu()
    p = O.SLSTMParams(t["W"], t["b"], t["R"])
    own = slstm_newton_ragged(p, t["x"], cs, max_iters=m["K"], picard_iters=m["P"], h0=t["h0"])
    e_ref = ((H - t["newton"]).abs() / (1 + t["newton"].abs())).max().item()
    e_own = ((H - own).abs() / (1 + own.abs())).max().item()
    print(f"  rel err vs reference {e_ref:.2e}, vs per-sequence oracle {e_own:.2e}", flush=True)
    assert e_ref <= 3e-5 and e_own <= 3e-5
    assert (H[..., 3, :] - t["newton"][..., 3, :]).abs().max().item() <= 1e-5
    assert torch.allclose(Hs, t["sequential"], rtol=0, atol=2e-5)


def test_gru_head_ragged_matches_reference():
    from pararnn_amd import ParaGRU, newton_apply, verify_agreement

    print("case gru head ragged fp32 (lengths 20, 45, 7)", flush=True)
    t, m = load_golden("gru_head_ragged_fp32")
    cell = ParaGRU(m["d_in"], m["d"], mix="head", n_heads=m["n_heads"])
    with torch.no_grad():
        for k in ("A_z", "A_r", "A_n"):
            getattr(cell, k).copy_(t[k])
        cell.W_x.weight.copy_(t["W"])
        cell.W_x.bias.copy_(t["b"])
    cell = cell.to(DEV)
    cs = t["cu_seqlens"].to(DEV)
    with torch.no_grad():
        H = newton_apply(cell, t["x"].to(DEV), _cfg(m["K"]), h0=t["h0"].to(DEV),
                         cu_seqlens=cs).cpu()
    err = (H - t["newton"]).abs().max().item()
    print(f"  max|gpu - reference| {err:.2e}", flush=True)
    assert err <= 1e-5
    rep = verify_agreement(cell, t["x"].to(DEV), config=_cfg(m["K"]), h0=t["h0"].to(DEV),
                           cu_seqlens=cs)
    print(f"  verify_agreement max_abs {rep.max_abs:.2e}", flush=True)
    assert rep.ok


def test_block_table_gathers_pool_rows():
    from pararnn_amd import NewtonConfig, ParaSLSTM, newton_apply

    print("case slstm block_table (pool of 6, batch 3) bf16", flush=True)
    torch.manual_seed(0)
    cell = ParaSLSTM(16, 64).to(DEV, torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 300, 16, generator=g).to(DEV, torch.bfloat16)
    pool = torch.randn(6, 4, 64, generator=g)
    pool[:, 1] = pool[:, 1].abs() + 0.5
    pool = pool.to(DEV, torch.bfloat16)
    bt = torch.tensor([4, 0, 4], device=DEV)
    cfg = NewtonConfig(max_iters=2, residual_fail=None)
    with torch.no_grad():
        a = newton_apply(cell, x, cfg, h0=pool, block_table=bt)
        b = newton_apply(cell, x, cfg, h0=pool[bt.long()])
    assert torch.equal(a, b)
    with pytest.raises(ValueError, match="outside pool"):
        with torch.no_grad():
            newton_apply(cell, x, cfg, h0=pool, block_table=torch.tensor([0, 1, 9], device=DEV))


def test_ragged_backward_equals_per_sequence_sum():
    from pararnn_amd import ParaSLSTM, newton_apply

    print("case slstm ragged backward fp32 vs per-sequence backward", flush=True)
    torch.manual_seed(2)
    cell = ParaSLSTM(8, 32).to(DEV)
    g = torch.Generator().manual_seed(3)
    lengths = [50, 13, 77]
    cs = torch.tensor([0, 50, 63, 140], device=DEV)
    x = torch.randn(1, 140, 8, generator=g).to(DEV)
    up = torch.randn(1, 140, 4, 32, generator=g).to(DEV)
    h0 = torch.randn(3, 4, 32, generator=g)
    h0[:, 1] = h0[:, 1].abs() + 0.5
    h0 = h0.to(DEV)
    cfg = _cfg(3, 3)
    xa = x.clone().requires_grad_(True)
    ha = h0.clone().requires_grad_(True)
    (newton_apply(cell, xa, cfg, h0=ha, cu_seqlens=cs) * up).sum().backward()
    ga = {n: p.grad.clone() for n, p in cell.named_parameters()}
    cell.zero_grad()
    xb = x.clone().requires_grad_(True)
    hb = h0.clone().requires_grad_(True)
    off = 0
    for s, n in enumerate(lengths):
        out = newton_apply(cell, xb[:, off:off + n], cfg, h0=hb[s:s + 1])
        (out * up[:, off:off + n]).sum().backward()
        off += n
    for name, p in cell.named_parameters():
        e = ((ga[name] - p.grad).abs().max() / p.grad.abs().max()).item()
        print(f"  grad {name}: rel diff {e:.2e}", flush=True)
        assert e <= 1e-5
    for name, a, b in (("x", xa.grad, xb.grad), ("h0", ha.grad, hb.grad)):
        e = ((a - b).abs().max() / b.abs().max()).item()
        print(f"  grad {name}: rel diff {e:.2e}", flush=True)
        assert e <= 1e-5


def _uneven(d_x, extra=(), seed=5):
    """Lengths that make three length groups (one rectangle would pad the
    short sequences ~40x)."""
    from pararnn_amd.ragged import RaggedPlan

    lengths = [2500, 31, 900, 700, 12, 60]
    cs = torch.tensor([0] + lengths).cumsum(0)
    assert RaggedPlan(cs, torch.device("cpu")).n_groups == 3
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, int(cs[-1]), d_x, generator=g)
    return lengths, cs, x, [torch.randn(len(lengths), *e, generator=g) for e in extra]


def test_slstm_ragged_length_groups(monkeypatch):
    """Uneven lengths: the packed stream solved in the kernels (default), and
    with PARARNN_AMD_PACKED=0 as several padded length groups, against the
    single padded rectangle (PARARNN_AMD_RAGGED_GROUPS=0): forward and every
    gradient; the forward also against the per-sequence oracle."""
    from pararnn_amd import ParaSLSTM, newton_apply

    print("case slstm ragged length groups fp32 (3 groups, lengths 12..2500)", flush=True)
    torch.manual_seed(4)
    cell = ParaSLSTM(8, 32).to(DEV)
    lengths, cs, x, (h0,) = _uneven(8, extra=((4, 32),))
    h0[:, 1] = h0[:, 1].abs() + 0.5
    up = torch.randn(1, x.shape[1], 4, 32, generator=torch.Generator().manual_seed(6))
    cfg = _cfg(3, 3)
    x, h0, up, csd = x.to(DEV), h0.to(DEV), up.to(DEV), cs.to(DEV)

    def run():
        cell.zero_grad(set_to_none=True)
        xx, hh = x.clone().requires_grad_(True), h0.clone().requires_grad_(True)
        H = newton_apply(cell, xx, cfg, h0=hh, cu_seqlens=csd)
        (H * up).sum().backward()
        out = {"H": H.detach(), "x": xx.grad, "h0": hh.grad}
        out.update({n: p.grad.clone() for n, p in cell.named_parameters()})
        return out

    packed = run()
    monkeypatch.setenv("PARARNN_AMD_PACKED", "0")
    grouped = run()
    monkeypatch.setenv("PARARNN_AMD_RAGGED_GROUPS", "0")
    single = run()
    for name, got in (("grouped", grouped), ("packed", packed)):
        for k in got:
            e = ((got[k] - single[k]).abs().max() / single[k].abs().max()).item()
            print(f"  {k}: {name} vs single rel diff {e:.2e}", flush=True)
            assert e <= 1e-5, (name, k)
    p = O.SLSTMParams(cell.W_x.weight.detach().cpu(), cell.W_x.bias.detach().cpu(),
                      cell.R.detach().cpu())
    own = slstm_newton_ragged(p, x.cpu(), cs, max_iters=3, picard_iters=3, h0=h0.cpu())
    for name, got in (("grouped", grouped), ("packed", packed)):
        e_own = ((got["H"].cpu() - own).abs() / (1 + own.abs())).max().item()
        print(f"  {name}: rel err vs per-sequence oracle {e_own:.2e}", flush=True)
        assert e_own <= 3e-5


def test_gru_head_ragged_length_groups(monkeypatch):
    """Head GRU, uneven lengths: the packed stream in the kernels (default),
    padded length groups (PARARNN_AMD_PACKED=0) and one padded rectangle
    (also PARARNN_AMD_RAGGED_GROUPS=0): forward and every gradient, and the
    forward against the per-sequence oracle."""
    from oracle.ragged import gru_head_newton_ragged

    from pararnn_amd import ParaGRU, newton_apply

    print("case gru head ragged length groups fp32 (3 groups, lengths 12..2500)", flush=True)
    torch.manual_seed(7)
    cell = ParaGRU(16, 128, mix="head", n_heads=2).to(DEV)
    lengths, cs, x, (h0,) = _uneven(16, extra=((128,),))
    up = torch.randn(1, x.shape[1], 128, generator=torch.Generator().manual_seed(8))
    x, h0, csd, up = x.to(DEV), (0.3 * h0).to(DEV), cs.to(DEV), up.to(DEV)

    def run():
        cell.zero_grad(set_to_none=True)
        xx, hh = x.clone().requires_grad_(True), h0.clone().requires_grad_(True)
        H = newton_apply(cell, xx, _cfg(3), h0=hh, cu_seqlens=csd)
        (H * up).sum().backward()
        out = {"H": H.detach(), "x": xx.grad, "h0": hh.grad}
        out.update({n: p.grad.clone() for n, p in cell.named_parameters()})
        return out

    packed = run()
    monkeypatch.setenv("PARARNN_AMD_PACKED", "0")
    grouped = run()
    monkeypatch.setenv("PARARNN_AMD_RAGGED_GROUPS", "0")
    single = run()
    for name, got in (("grouped", grouped), ("packed", packed)):
        for k in got:
            e = ((got[k] - single[k]).abs().max() / single[k].abs().max()).item()
            print(f"  {k}: {name} vs single rel diff {e:.2e}", flush=True)
            assert e <= 1e-5, (name, k)
    p = O.GRUHeadParams(cell.W_x.weight.detach().cpu(), cell.W_x.bias.detach().cpu(),
                        *(a.detach().cpu() for a in cell.clipped_a_head()))
    own = gru_head_newton_ragged(p, x.cpu(), cs, max_iters=3, h0=h0.cpu())
    err = (packed["H"].cpu() - own).abs().max().item()
    print(f"  packed: max|gpu - per-sequence oracle| {err:.2e}", flush=True)
    assert err <= 1e-5


def test_fused_newton_cu_seqlens_with_block_table():
    """Packed sequences with a paged h0: packed sequence s reads pool row
    block_table[s] (kernels/_fused_common.py:56, newton_cfc.py:357), the same
    result as the gathered dense h0."""
    from pararnn_amd import ParaSLSTM, fused_newton

    print("case slstm fused_newton cu_seqlens + block_table (6 sequences, pool of 8)", flush=True)
    torch.manual_seed(8)
    cell = ParaSLSTM(8, 32).to(DEV)
    g = torch.Generator().manual_seed(9)
    lengths, cs, x, (pool,) = _uneven(8, extra=((4, 32),))
    pool = torch.randn(len(lengths) + 2, 4, 32, generator=g)
    pool[:, 1] = pool[:, 1].abs() + 0.5
    pool, csd = pool.to(DEV), cs.to(DEV)
    bt = torch.tensor([6, 0, 3, 3, 7, 1], device=DEV)
    # The default look-back composes whichever predecessors have published, so
    # two solves of the same inputs may differ in the last bits; the
    # deterministic walk makes them bit-identical, which is the bar here.
    prev = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True, warn_only=True)
    try:
        with torch.no_grad():
            wx = cell.W_x(x.to(DEV))
            a = fused_newton(cell, wx, max_iters=2, omega=1.0, h0=pool, picard_iters=3,
                             cu_seqlens=csd, block_table=bt)
            b = fused_newton(cell, wx, max_iters=2, omega=1.0, h0=pool[bt], picard_iters=3,
                             cu_seqlens=csd)
    finally:
        torch.use_deterministic_algorithms(prev)
    err = ((a - b).abs().max() / b.abs().max()).item()
    print(f"  rel diff paged vs gathered h0 {err:.2e}", flush=True)
    assert torch.equal(a, b)
    with pytest.raises(ValueError, match="block_table B=2"):
        with torch.no_grad():
            fused_newton(cell, wx, max_iters=2, omega=1.0, h0=pool, cu_seqlens=csd,
                         block_table=bt[:2])
