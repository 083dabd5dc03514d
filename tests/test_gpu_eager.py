"""NewtonConfig(scan_backend='eager') on the GPU: the reference's eager Newton
loop (solvers/newton/__init__.py:467-549), whose ParaSLSTM iterations round
like the eager tensor ops (cell and Jacobian op by op in the tensor dtype,
cells/para_slstm.py:241-281 and :378-446; fp32 scan, solvers/scan.py:229-246;
rounded update), checked against the reference's own eager golden vectors and
the oracle's eager restatement.  Every case prints its name before running."""

import pytest
import torch
from conftest import load_golden

import oracle as O

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("lookback_mode")]

DEV = "cuda:0"


def _cfg(K, P, **kw):
    from pararnn_amd import NewtonConfig

    kw.setdefault("residual_atol", None)
    return NewtonConfig(max_iters=K, picard_iters=P, residual_fail=None, picard_adapt=False,
                        scan_backend="eager", **kw)


def _cell(t, m, dtype):
    from pararnn_amd import ParaSLSTM

    cell = ParaSLSTM(m["d_in"], m["d"], mix="diag")
    with torch.no_grad():
        cell.W_x.weight.copy_(t["W"])
        cell.W_x.bias.copy_(t["b"])
        cell.R.copy_(t["R"])
    return cell.to(device=DEV, dtype=dtype)


def _rel(got, ref):
    """Per slot (max |got - ref| / max |ref|, ||got - ref|| / ||ref||)."""
    got, ref = got.double().cpu(), ref.double().cpu()
    return [(((got[..., k, :] - ref[..., k, :]).abs().max() / ref[..., k, :].abs().max()).item(),
             ((got[..., k, :] - ref[..., k, :]).norm() / ref[..., k, :].norm()).item())
            for k in range(4)]


@pytest.mark.parametrize("name", ["slstm_bf16", "slstm_fp16"])
def test_narrow_dtypes_match_reference_eager_output(name):
    """north_star's bf16 bar, <= 2e-2 relative against the reference's eager
    Newton output (golden ``newton``, same seed, same K and P), on every slot
    (the h slot is the layer output), through newton_apply end to end (its
    W_x GEMM on the GPU) and from the golden wx."""
    from pararnn_amd import newton_apply

    print(f"case eager {name} vs reference eager golden", flush=True)
    t, m = load_golden(name)
    dtype = torch.bfloat16 if m["dtype"] == "bfloat16" else torch.float16
    cell = _cell(t, m, dtype)
    h0 = t["h0"].to(DEV) if "h0" in t else None
    with torch.no_grad():
        out = newton_apply(cell, t["x"].to(DEV), _cfg(m["K"], m["P"]), h0=h0).float().cpu()
        cfg_wx = _cfg(m["K"], m["P"])
        from pararnn_amd.newton import _newton_eager

        out_wx = _newton_eager(cell, t["wx"].to(DEV), cfg_wx, h0=h0)[0].float().cpu()
    eager = t["newton"].float()
    for tag, got in (("newton_apply", out), ("golden wx", out_wx)):
        rows = _rel(got, eager)
        print(f"  {tag}: per slot (c,n,m,h) max/norm rel "
              + str([f"{a:.2e}/{b:.2e}" for a, b in rows]), flush=True)
        assert max(a for a, _ in rows) <= 2e-2
        assert max(b for _, b in rows) <= 2e-2
    # the bf16 ulp structure: most elements land on the reference's value
    same = (out_wx == eager).double().mean().item()
    print(f"  golden wx: fraction of elements equal to the reference's {same:.4f}", flush=True)
    assert same >= 0.9


def test_eager_is_closer_to_reference_eager_than_fused():
    """The reason the eager backend exists: at the golden case the fused
    semantics sit ~3% from the reference's eager output on the h slot; the
    eager rounding brings the GPU result within a fraction of that."""
    from pararnn_amd import fused_newton
    from pararnn_amd.newton import _newton_eager

    print("case eager vs fused distance to reference eager (slstm_bf16)", flush=True)
    t, m = load_golden("slstm_bf16")
    cell = _cell(t, m, torch.bfloat16)
    wx = t["wx"].to(DEV)
    with torch.no_grad():
        eager_gpu = _newton_eager(cell, wx, _cfg(m["K"], m["P"]), h0=None)[0].float().cpu()
        fused_gpu = fused_newton(cell, wx, max_iters=m["K"], omega=1.0, h0=None,
                                 picard_iters=m["P"]).float().cpu()
    ref = t["newton"].float()
    d_e = (eager_gpu[..., 3, :] - ref[..., 3, :]).norm() / ref[..., 3, :].norm()
    d_f = (fused_gpu[..., 3, :] - ref[..., 3, :]).norm() / ref[..., 3, :].norm()
    print(f"  h slot norm-rel: eager {d_e:.2e}, fused {d_f:.2e}", flush=True)
    assert d_e <= 0.25 * d_f


@pytest.mark.parametrize("B,T,d,K,P,dtype", [
    (1, 1, 1, 1, 0, torch.bfloat16), (2, 70, 5, 2, 2, torch.bfloat16),
    (3, 129, 70, 3, 1, torch.bfloat16), (1, 1000, 130, 2, 3, torch.bfloat16),
    (2, 333, 64, 2, 3, torch.float16), (2, 200, 33, 3, 1, torch.float32),
])
def test_ragged_shapes_vs_oracle_eager(B, T, d, K, P, dtype):
    """Partial tiles, d not a multiple of 64, T = 1, with h0: the GPU eager
    loop against the oracle's eager restatement (which reproduces the
    reference's eager goldens bit for bit).  Narrow dtypes: the values agree
    up to rounding-boundary flips (fp32 sums in another order), so most
    elements are equal and the rest are close; fp32: within 1e-4 of
    1 + |x|."""
    from pararnn_amd import ParaSLSTM, newton_apply

    print(f"case eager ragged B={B} T={T} d={d} K={K} P={P} {dtype}", flush=True)
    torch.manual_seed(B * 1000 + T + d + 3)
    cell = ParaSLSTM(7, d).to(dtype)
    x = torch.randn(B, T, 7).to(dtype)
    h0 = torch.randn(B, 4, d) * 0.5
    h0[:, 1] = h0[:, 1].abs() + 0.5
    h0 = h0.to(dtype)
    p = O.SLSTMParams(cell.W_x.weight.detach(), cell.W_x.bias.detach(), cell.R.detach())
    with torch.no_grad():
        wx = p.wx(x)
        ref = O.slstm_newton(p, None, max_iters=K, picard_iters=P, h0=h0, wx=wx, work="eager")
        from pararnn_amd.newton import _newton_eager

        cell = cell.to(DEV)
        out = _newton_eager(cell, wx.to(DEV), _cfg(K, P), h0=h0.to(DEV))[0].cpu()
        out2 = newton_apply(cell, x.to(DEV), _cfg(K, P), h0=h0.to(DEV)).cpu()
    assert out.dtype == dtype and out2.shape == out.shape
    if dtype == torch.float32:
        err = ((out - ref).abs() / (1 + ref.abs())).max().item()
        print(f"  max rel vs oracle eager {err:.2e}", flush=True)
        assert err <= 1e-4
        return
    same = (out == ref).double().mean().item()
    err = ((out.float() - ref.float()).norm() / ref.float().norm()).item()
    print(f"  equal fraction {same:.4f}, norm-rel {err:.2e}", flush=True)
    assert same >= 0.9 and err <= 1e-2


def test_fp32_eager_vs_reference_golden():
    """fp32: the eager loop's arithmetic is the fused path's up to operation
    order; the h slot within 1e-5 of the reference's eager output, every slot
    within the reference's own fp32 error of the float64 iterate."""
    from pararnn_amd import newton_apply
    from oracle.slstm import slstm_newton_f64

    print("case eager fp32 slstm_cfg1_fp32", flush=True)
    t, m = load_golden("slstm_cfg1_fp32")
    cell = _cell(t, m, torch.float32)
    with torch.no_grad():
        out = newton_apply(cell, t["x"].to(DEV), _cfg(m["K"], m["P"])).cpu().double()
    p = O.SLSTMParams(t["W"], t["b"], t["R"])
    _, exact = slstm_newton_f64(p, p.wx(t["x"]), max_iters=m["K"], picard_iters=m["P"])
    ref = t["newton"].double()
    exact = exact.double()
    d_ref = (out - ref).abs()
    e_ours = (out - exact).abs() / (1 + exact.abs())
    print(f"  |gpu-ref| per slot {['%.1e' % d_ref[..., k, :].max() for k in range(4)]}; "
          f"own rel error {e_ours.max().item():.1e}", flush=True)
    assert d_ref[..., 3, :].max().item() <= 1e-5
    assert e_ours.max().item() <= 3e-5


def test_early_stop_counts_the_checked_iteration():
    """With residual_atol the eager loop reads max|F| of the iterate before
    each update and stops below the bar; that iteration counts
    (newton/__init__.py:516-533).  The result equals the eager loop run for
    one update fewer than the count."""
    from pararnn_amd import NewtonStats, newton_apply

    print("case eager early stop (slstm_h0_fp32, atol 1e-4)", flush=True)
    t, m = load_golden("slstm_h0_fp32")
    cell = _cell(t, m, torch.float32)
    x, h0 = t["x"].to(DEV), t["h0"].to(DEV)
    st = NewtonStats()
    with torch.no_grad():
        out = newton_apply(cell, x, _cfg(8, m["P"], residual_atol=1e-4), h0=h0, stats=st)
        same = newton_apply(cell, x, _cfg(st.iters - 1, m["P"]), h0=h0)
    print(f"  iters {st.iters}, history {['%.1e' % v for v in st.residual_history]}, "
          f"backend {st.scan_backend}", flush=True)
    assert st.scan_backend == "eager"
    assert 2 <= st.iters < 8 and len(st.residual_history) == st.iters
    assert st.residual_history[-1] < 1e-4 <= min(st.residual_history[:-1])
    assert st.max_residual == st.residual_history[-1]
    assert (out - same).abs().max().item() <= 1e-6 * (1 + same.abs().max().item())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_packed_stream_vs_each_sequence_alone(dtype):
    """cu_seqlens with the eager backend: the packed kernel cuts the carry at
    every head and starts each sequence from its own h0 row."""
    from pararnn_amd import ParaSLSTM, newton_apply

    print(f"case eager packed stream {dtype}", flush=True)
    torch.manual_seed(21)
    lengths = [257, 1, 64, 300, 90]
    cs = torch.tensor([0] + lengths).cumsum(0).to(torch.int32)
    d = 80
    cell = ParaSLSTM(9, d).to(dtype)
    x = torch.randn(1, int(cs[-1]), 9).to(dtype)
    h0 = torch.randn(len(lengths), 4, d) * 0.5
    h0[:, 1] = h0[:, 1].abs() + 0.5
    h0 = h0.to(dtype)
    cell = cell.to(DEV)
    cfg = _cfg(2, 3)
    with torch.no_grad():
        out = newton_apply(cell, x.to(DEV), cfg, h0=h0.to(DEV), cu_seqlens=cs.to(DEV)).cpu()
        alone = [newton_apply(cell, x[:, a:b].to(DEV), cfg, h0=h0[s:s + 1].to(DEV)).cpu()
                 for s, (a, b) in enumerate(zip(cs[:-1].tolist(), cs[1:].tolist()))]
    ref = torch.cat(alone, dim=1)
    err = ((out.float() - ref.float()).norm() / ref.float().norm()).item()
    same = (out == ref).double().mean().item()
    print(f"  norm-rel {err:.2e}, equal fraction {same:.4f}", flush=True)
    assert err <= (1e-5 if dtype == torch.float32 else 1e-2)


def test_gru_head_eager_meets_the_bf16_bar():
    """ParaGRU(mix='head') under 'eager' runs the fused kernels: its eager and
    fused semantics agree within the bf16 tolerance (reference eager golden
    ``gru_head_bf16['newton']``, K=3)."""
    from pararnn_amd import NewtonStats, ParaGRU, newton_apply

    print("case eager gru head bf16", flush=True)
    t, m = load_golden("gru_head_bf16")
    cell = ParaGRU(m["d_in"], m["n_heads"] * m["d_head"], mix="head", n_heads=m["n_heads"])
    with torch.no_grad():
        cell.W_x.weight.copy_(t["W"])
        cell.W_x.bias.copy_(t["b"])
        for k in ("A_z", "A_r", "A_n"):
            getattr(cell, k).copy_(t[k])
    cell = cell.to(DEV, torch.bfloat16)
    st = NewtonStats()
    with torch.no_grad():
        out = newton_apply(cell, t["x"].to(DEV), _cfg(m["K"], 0), stats=st).float().cpu()
    ref = t["newton"].float()
    rel = ((out - ref).abs().max() / ref.abs().max()).item()
    print(f"  max rel vs reference eager {rel:.2e}; backend {st.scan_backend}", flush=True)
    assert st.scan_backend == "eager" and rel <= 2e-2


def test_gru_head_eager_early_stop():
    """Head GRU with residual_atol: the iterate before update k is the K = k
    solve, so the loop stops at the first k whose residual is below the bar."""
    from pararnn_amd import NewtonStats, ParaGRU, newton_apply

    print("case eager gru head early stop", flush=True)
    torch.manual_seed(5)
    cell = ParaGRU(16, 128, mix="head", n_heads=2).to(DEV)
    x = torch.randn(2, 300, 16, device=DEV)
    st = NewtonStats()
    with torch.no_grad():
        out = newton_apply(cell, x, _cfg(6, 0, residual_atol=1e-5), stats=st)
        same = newton_apply(cell, x, _cfg(st.iters - 1, 0))
    print(f"  iters {st.iters}, history {['%.1e' % v for v in st.residual_history]}",
          flush=True)
    assert st.residual_history[-1] < 1e-5 and len(st.residual_history) == st.iters
    assert torch.equal(out, same)


def test_gradients_through_the_eager_solve():
    """Autograd through an eager solve uses the eq. 2.6 backward at the eager
    H* (the reference's backward does not depend on how H* was found beyond
    its rounding): gradients match the same backward run at the fused H*
    within the bf16 sensitivity of the two trajectories."""
    from pararnn_amd import NewtonConfig, ParaSLSTM, newton_apply

    print("case eager autograd fp32", flush=True)
    torch.manual_seed(9)
    cell = ParaSLSTM(6, 40).to(DEV)
    x = torch.randn(2, 150, 6, device=DEV)
    up = torch.randn(2, 150, 4, 40, device=DEV)
    grads = {}
    for backend in ("eager", "fused"):
        cfg = NewtonConfig(max_iters=4, picard_iters=3, residual_atol=None, residual_fail=None,
                           picard_adapt=False, scan_backend=backend)
        cell.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_(True)
        newton_apply(cell, xx, cfg).backward(up)
        grads[backend] = (xx.grad.clone(), cell.R.grad.clone(), cell.W_x.weight.grad.clone())
    for a, b in zip(grads["eager"], grads["fused"]):
        rel = ((a - b).norm() / b.norm()).item()
        print(f"  eager vs fused gradient norm-rel {rel:.2e}", flush=True)
        assert rel <= 1e-4


def test_block_table_needs_fused():
    from pararnn_amd import ParaSLSTM, newton_apply

    cell = ParaSLSTM(4, 8).to(DEV)
    x = torch.randn(2, 5, 4, device=DEV)
    pool = torch.zeros(3, 4, 8, device=DEV)
    with pytest.raises(ValueError, match="block_table"):
        with torch.no_grad():
            newton_apply(cell, x, _cfg(2, 1), h0=pool,
                         block_table=torch.tensor([0, 2], dtype=torch.int32, device=DEV))


def test_fp16_packed_stream_with_early_stop():
    """fp16 storage, a packed stream with per-sequence h0, and the residual-gated
    early stop: the count and the result agree with the fixed-K eager loop at
    that count, and each sequence stays close to being solved alone."""
    from pararnn_amd import NewtonStats, ParaSLSTM, newton_apply

    print("case eager fp16 packed early stop", flush=True)
    torch.manual_seed(8)
    lengths = [100, 1, 260, 33]
    cs = torch.tensor([0] + lengths).cumsum(0).to(torch.int32).to(DEV)
    d = 70
    cell = ParaSLSTM(6, d).to(DEV, torch.float16)
    x = torch.randn(1, int(cs[-1]), 6, device=DEV).to(torch.float16)
    h0 = torch.randn(len(lengths), 4, d, device=DEV) * 0.5
    h0[:, 1] = h0[:, 1].abs() + 0.5
    h0 = h0.to(torch.float16)
    st = NewtonStats()
    with torch.no_grad():
        # zero-hidden guess (P = 0), so the stop takes a few iterations
        out = newton_apply(cell, x, _cfg(8, 0, residual_atol=5e-2), h0=h0, cu_seqlens=cs,
                           stats=st)
        same = newton_apply(cell, x, _cfg(st.iters - 1, 0), h0=h0, cu_seqlens=cs)
        alone = torch.cat([newton_apply(cell, x[:, a:b], _cfg(st.iters - 1, 0), h0=h0[s:s + 1])
                           for s, (a, b) in enumerate(zip(cs[:-1].tolist(), cs[1:].tolist()))],
                          dim=1)
    print(f"  iters {st.iters}, history {['%.1e' % v for v in st.residual_history]}", flush=True)
    assert st.iters >= 2 and len(st.residual_history) == st.iters
    assert st.residual_history[-1] < 5e-2 <= min(st.residual_history[:-1])
    d_same = ((out.float() - same.float()).norm() / same.float().norm()).item()
    d_alone = ((out.float() - alone.float()).norm() / alone.float().norm()).item()
    print(f"  vs fixed K: {d_same:.2e}; vs each sequence alone: {d_alone:.2e}", flush=True)
    assert d_same <= 1e-3 and d_alone <= 1e-2
