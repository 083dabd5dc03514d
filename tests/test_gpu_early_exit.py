"""NewtonConfig(fused_early_exit=True) for ParaSLSTM(mix='diag'): the fused
iterations one at a time on the fp32 work iterate, the host reading max|F| of
the rounded iterate after each and stopping below residual_atol (reference
solvers/newton/__init__.py:696-762, kernels/newton_slstm.py:2892-2922).
Checked against the CPU oracle at the iteration count the exit chose.  Every
case prints its name before running."""

import pytest
import torch
from conftest import load_golden

import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _cell(t, m, dtype):
    from pararnn_amd import ParaSLSTM

    cell = ParaSLSTM(m["d_in"], m["d"], mix="diag")
    with torch.no_grad():
        cell.W_x.weight.copy_(t["W"])
        cell.W_x.bias.copy_(t["b"])
        cell.R.copy_(t["R"])
    return cell.to(device=DEV, dtype=dtype)


def test_early_exit_fp32_matches_oracle_at_the_exit_iteration():
    from pararnn_amd import NewtonConfig, NewtonStats, newton_apply

    print("case fused_early_exit fp32 (slstm_h0_fp32, atol 1e-4, max_iters 8)", flush=True)
    t, m = load_golden("slstm_h0_fp32")
    cell = _cell(t, m, torch.float32)
    cfg = NewtonConfig(max_iters=8, picard_iters=m["P"], residual_atol=1e-4, residual_fail=None,
                       picard_adapt=False, fused_early_exit=True)
    st = NewtonStats()
    with torch.no_grad():
        out = newton_apply(cell, t["x"].to(DEV), cfg, h0=t["h0"].to(DEV), stats=st).cpu()
    print(f"  iters {st.iters}, residual history {['%.2e' % r for r in st.residual_history]}",
          flush=True)
    assert 1 <= st.iters < 8
    assert len(st.residual_history) == st.iters
    assert st.residual_history[-1] < 1e-4 <= min(st.residual_history[:-1] + (1.0,))
    p = O.SLSTMParams(t["W"], t["b"], t["R"])
    ref = O.slstm_newton(p, t["x"], max_iters=st.iters, picard_iters=m["P"], h0=t["h0"])
    err = (out - ref).abs() / (1 + ref.abs())
    print(f"  max rel |gpu - oracle(K={st.iters})| {err.max().item():.2e}", flush=True)
    assert err.max().item() <= 1e-4


def test_early_exit_bf16_equals_the_fused_call_with_that_k():
    from pararnn_amd import NewtonConfig, NewtonStats, fused_newton, newton_apply

    print("case fused_early_exit bf16 (slstm_bf16, atol 5e-2)", flush=True)
    t, m = load_golden("slstm_bf16")
    cell = _cell(t, m, torch.bfloat16)
    cfg = NewtonConfig(max_iters=6, picard_iters=m["P"], residual_atol=5e-2, residual_fail=None,
                       picard_adapt=False, fused_early_exit=True)
    st = NewtonStats()
    x = t["x"].to(DEV)
    with torch.no_grad():
        out = newton_apply(cell, x, cfg, stats=st).float()
        ref = fused_newton(cell, cell.W_x(x), max_iters=st.iters, omega=1.0, h0=None,
                           picard_iters=m["P"]).float()
    rel = ((out - ref).norm() / ref.norm()).item()
    print(f"  iters {st.iters}; norm-rel vs the fused K={st.iters} call {rel:.2e}", flush=True)
    assert st.iters <= 6 and rel <= 1e-3


def test_early_exit_runs_all_iterations_when_the_bar_is_not_reached():
    from pararnn_amd import NewtonConfig, NewtonStats, newton_apply

    print("case fused_early_exit unreachable atol", flush=True)
    t, m = load_golden("slstm_cfg1_fp32")
    cell = _cell(t, m, torch.float32)
    cfg = NewtonConfig(max_iters=2, picard_iters=m["P"], residual_atol=1e-30, residual_fail=None,
                       picard_adapt=False, fused_early_exit=True)
    st = NewtonStats()
    with torch.no_grad():
        out = newton_apply(cell, t["x"].to(DEV), cfg, stats=st).cpu()
    assert st.iters == 2 and len(st.residual_history) == 2
    assert (out[..., 3, :] - t["newton"][..., 3, :]).abs().max().item() <= 1e-5


def test_early_exit_is_diag_slstm_only():
    from pararnn_amd import NewtonConfig, ParaGRU, newton_apply

    cell = ParaGRU(8, 64, mix="head", n_heads=1).to(DEV)
    cfg = NewtonConfig(max_iters=2, residual_atol=1e-4, fused_early_exit=True)
    with pytest.raises(TypeError, match="mix='diag' only"):
        with torch.no_grad():
            newton_apply(cell, torch.randn(1, 10, 8, device=DEV), cfg)


def _packed_case(dtype):
    from pararnn_amd import ParaSLSTM

    torch.manual_seed(11)
    lengths = [300, 1, 77, 200, 64]
    cs = torch.tensor([0] + lengths).cumsum(0).to(torch.int32)
    d = 96
    cell = ParaSLSTM(12, d)
    x = torch.randn(1, int(cs[-1]), 12)
    h0 = torch.randn(len(lengths), 4, d) * 0.5
    h0[:, 1] = h0[:, 1].abs() + 0.5
    return cell, x.to(dtype), h0.to(dtype), cs, lengths


@pytest.mark.parametrize("paged", [False, True], ids=["dense_h0", "block_table"])
def test_early_exit_on_a_packed_stream(paged):
    """fused_early_exit on a packed cu_seqlens stream runs in the packed
    kernels (heads cut the carry, each reads its own h0 row, or the pool row
    block_table names): the exit iteration is the first whose max|F| over the
    whole stream is below residual_atol, and the result equals the packed
    fused solve at that K and each sequence solved alone by the oracle."""
    from pararnn_amd import NewtonConfig, NewtonStats, fused_newton, newton_apply

    print(f"case fused_early_exit packed fp32 paged={paged}", flush=True)
    cell, x, h0, cs, lengths = _packed_case(torch.float32)
    p = O.SLSTMParams(cell.W_x.weight.detach(), cell.W_x.bias.detach(), cell.R.detach())
    cell = cell.to(DEV)
    # zero-hidden guess only (P = 0), so the exit takes a few iterations
    cfg = NewtonConfig(max_iters=8, picard_iters=0, residual_atol=1e-4, residual_fail=None,
                       picard_adapt=False, fused_early_exit=True)
    st = NewtonStats()
    csd = cs.to(DEV)
    if paged:
        pool = torch.randn(9, 4, cell.d_h) * 0.5
        pool[:, 1] = pool[:, 1].abs() + 0.5
        table = torch.tensor([7, 2, 5, 0, 3], dtype=torch.int32)
        pool[table.long()] = h0
        h0_arg, bt = pool.to(DEV), table.to(DEV)
    else:
        h0_arg, bt = h0.to(DEV), None
    with torch.no_grad():
        out = newton_apply(cell, x.to(DEV), cfg, h0=h0_arg, stats=st, cu_seqlens=csd,
                           block_table=bt).cpu()
        same_k = fused_newton(cell, cell.W_x(x.to(DEV)), max_iters=st.iters, omega=1.0,
                              h0=h0_arg, picard_iters=0, cu_seqlens=csd, block_table=bt).cpu()
    print(f"  iters {st.iters}, residual history {['%.2e' % r for r in st.residual_history]}",
          flush=True)
    assert 2 <= st.iters < 8 and len(st.residual_history) == st.iters
    assert st.residual_history[-1] < 1e-4 <= min(st.residual_history[:-1])
    d_same = (out - same_k).abs().max().item()
    print(f"  max|early exit - packed fused K={st.iters}| {d_same:.2e}", flush=True)
    assert d_same <= 1e-5 * (1 + same_k.abs().max().item())
    worst = 0.0
    for s, (a, b) in enumerate(zip(cs[:-1].tolist(), cs[1:].tolist())):
        ref = O.slstm_newton(p, x[:, a:b], max_iters=st.iters, picard_iters=0, h0=h0[s:s + 1])
        worst = max(worst, ((out[:, a:b] - ref).abs() / (1 + ref.abs())).max().item())
    print(f"  max rel vs each sequence alone (oracle) {worst:.2e}", flush=True)
    assert worst <= 1e-4


def test_early_exit_with_length_groups_is_refused():
    """With PARARNN_AMD_PACKED=0 a packed stream runs as padded length groups,
    where an exit decided per group would not be the stream's: the request is
    refused instead of dropped."""
    from pararnn_amd import NewtonConfig, newton_apply

    cell, x, h0, cs, _ = _packed_case(torch.float32)
    cfg = NewtonConfig(max_iters=4, picard_iters=3, residual_atol=1e-4, residual_fail=None,
                       picard_adapt=False, fused_early_exit=True)
    mp = pytest.MonkeyPatch()
    mp.setenv("PARARNN_AMD_PACKED", "0")
    try:
        with pytest.raises(ValueError, match="fused_early_exit"):
            with torch.no_grad():
                newton_apply(cell.to(DEV), x.to(DEV), cfg, h0=h0.to(DEV), cu_seqlens=cs.to(DEV))
    finally:
        mp.undo()
