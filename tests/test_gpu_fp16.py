"""fp16 storage on the GPU (the reference admits float16 wherever it admits
bfloat16: kernels/precision.py:20-34, fp32 algebra on narrow DRAM).  The same
bars as the bf16 tests, against the reference's eager fp16 golden vectors
(which the oracle reproduces bit for bit) and the oracle's fused-op
semantics.  Every case prints its name before running."""

import pytest
import torch
from conftest import load_golden

import oracle as O
from oracle.backward import slstm_backward

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("lookback_mode")]

DEV = "cuda:0"
F16 = torch.float16


def _cfg(K, P=None):
    from pararnn_amd import NewtonConfig

    return NewtonConfig(max_iters=K, picard_iters=P, residual_atol=None, residual_fail=None,
                        picard_adapt=False)


def _slstm_cell(t, m):
    from pararnn_amd import ParaSLSTM

    cell = ParaSLSTM(m["d_in"], m["d"], mix="diag")
    with torch.no_grad():
        cell.W_x.weight.copy_(t["W"])
        cell.W_x.bias.copy_(t["b"])
        cell.R.copy_(t["R"])
    return cell.to(device=DEV, dtype=F16)


def _ulps(got, ref):
    """|got - ref| in fp16 ulps of ref (normal range; subnormals at 2^-24)."""
    got, ref = got.double().cpu(), ref.double().cpu()
    e = torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14)))
    return (got - ref).abs() / torch.exp2(e - 10)


def test_slstm_init_matches_reference_eager_bits():
    """The single-launch warm start against the reference's eager fp16
    ``slstm_picard_init`` (solvers/slstm_picard.py:143-181), from h0: each
    pass's state is rounded to fp16 once from fp32 algebra, so the kernel lands
    on the same fp16 values up to rounding-boundary flips of one ulp."""
    from pararnn_amd import slstm_init_fused

    print("case slstm_fp16 init vs reference eager fp16", flush=True)
    t, m = load_golden("slstm_fp16")
    cell = _slstm_cell(t, m)
    with torch.no_grad():
        got = slstm_init_fused(t["wx"].to(DEV), cell.clipped_r(), t["h0"].to(DEV),
                               picard_iters=m["P"], eps=cell.eps).float().cpu()
    ref = t["init"].float()
    u = _ulps(got, ref)
    per = [(u[..., k, :].max().item(), (u[..., k, :] > 0).double().mean().item())
           for k in range(4)]
    print("  per slot (c,n,m,h): max ulp / frac differing "
          + str([f"{a:.0f}/{b:.1e}" for a, b in per]), flush=True)
    assert u.max().item() <= 2
    assert (u > 0).double().mean().item() <= 1e-3


def test_slstm_newton_matches_fused_semantics_and_reference():
    """K Newton iterations in fp32 work on fp16 storage (the reference's fused
    op: kernels/newton_slstm.py:2780-2939, _fused_common.py:171-183) against
    the oracle's ``work='fused'`` evaluation of the same algorithm, and the h
    slot against the reference's eager fp16 solve no further than the fused
    semantics itself is (+10%)."""
    from pararnn_amd import fused_newton, newton_apply

    print("case slstm_fp16 newton", flush=True)
    t, m = load_golden("slstm_fp16")
    cell = _slstm_cell(t, m)
    h0 = t["h0"].to(DEV)
    with torch.no_grad():
        out = fused_newton(cell, t["wx"].to(DEV), max_iters=m["K"], omega=1.0, h0=h0,
                           picard_iters=m["P"]).float().cpu()
        out2 = newton_apply(cell, t["x"].to(DEV), _cfg(m["K"], m["P"]), h0=h0).float().cpu()
    p = O.SLSTMParams(t["W"], t["b"], t["R"])
    fused = O.slstm_newton(p, None, max_iters=m["K"], picard_iters=m["P"], wx=t["wx"],
                           h0=t["h0"], work="fused").float()
    eager = t["newton"].float()
    rel = [((out[..., k, :] - fused[..., k, :]).abs().max()
            / fused[..., k, :].abs().max()).item() for k in range(4)]
    print("  vs fused semantics per slot max rel " + str([f"{v:.1e}" for v in rel]), flush=True)
    assert max(rel) <= 2e-3

    def nrel(a, b):
        return ((a - b).norm() / b.norm()).item()

    g_h, f_h = nrel(out[..., 3, :], eager[..., 3, :]), nrel(fused[..., 3, :], eager[..., 3, :])
    print(f"  h slot vs reference eager fp16: gpu norm-rel {g_h:.2e}, fused semantics {f_h:.2e}",
          flush=True)
    assert g_h <= 1.1 * f_h + 1e-4
    assert nrel(out2, out) <= 2e-3


def test_slstm_backward_op_matches_float64():
    """The eq. 2.6 reverse kernel on fp16 operands at the reference's H*: fp32
    work, g_wx rounded to fp16 once."""
    from pararnn_amd import ops

    print("case slstm_bwd_fp16 op vs float64", flush=True)
    t, m = load_golden("slstm_bwd_fp16")
    p = O.SLSTMParams(t["W"], t["b"], t["R"])
    wx = p.wx(t["x"])
    p64 = O.SLSTMParams(t["W"].double(), t["b"].double(), t["R"].double())
    ex = slstm_backward(p64, t["x"].double(), t["newton"].double(), t["grad"].double(), None,
                        work=torch.float64, wx=wx.double())
    g_wx, g_r, _, g_b = ops.slstm_backward_fused(wx.to(DEV), p.r().to(DEV), None,
                                                 t["newton"].to(DEV), t["grad"].to(DEV),
                                                 eps=m["eps"])
    assert g_wx.dtype == F16

    def rel(a, b):
        a, b = a.double().cpu(), b.double().cpu()
        return ((a - b).abs().max() / b.abs().max()).item()

    e_wx, e_b = rel(g_wx, ex["g_wx"]), rel(g_b.reshape(-1), ex["b"])
    print(f"  g_wx rel {e_wx:.2e}  g_b rel {e_b:.2e}", flush=True)
    assert e_wx <= 1e-3 and e_b <= 1e-4


def test_slstm_autograd_at_reference_trajectory():
    """newton_apply's backward in fp16 against the reference's eager fp16
    gradients, the forward taken at the reference's own H* (the backward alone;
    H* of the two forwards differ by fp16 rounding of the work)."""
    from pararnn_amd.newton import _eq26_vjp

    print("case slstm_bwd_fp16 at the reference's H* vs the reference's gradients", flush=True)
    t, m = load_golden("slstm_bwd_fp16")
    cell = _slstm_cell(t, m)
    with torch.no_grad():
        gx, pg, _ = _eq26_vjp(cell, t["newton"].to(DEV), t["x"].to(DEV), t["grad"].to(DEV))
    names = {"R": "R", "W_x.weight": "W", "W_x.bias": "b"}
    ours = dict(x=gx, **{names[n]: g for (n, _), g in zip(cell.named_parameters(), pg)})
    for k, g in ours.items():
        ref = t[f"grad_{k}"].float()
        nrel = ((g.float().cpu() - ref).norm() / ref.norm()).item()
        print(f"  grad_{k}: norm-rel vs reference eager fp16 {nrel:.3e}", flush=True)
        assert g.dtype == F16 and nrel <= 5e-3, k


def _gru_cell(t, m):
    from pararnn_amd import ParaGRU

    cell = ParaGRU(m["d_in"], m["n_heads"] * m["d_head"], mix="head", n_heads=m["n_heads"])
    with torch.no_grad():
        cell.W_x.weight.copy_(t["W"])
        cell.W_x.bias.copy_(t["b"])
        for k in ("A_z", "A_r", "A_n"):
            getattr(cell, k).copy_(t[k])
    return cell.to(device=DEV, dtype=F16)


@pytest.mark.parametrize("mfma_replay", ["0", "1"])
def test_gru_head_matches_fused_semantics_and_reference(mfma_replay, monkeypatch):
    """Head GRU, fp16 storage: against the oracle's fp32 algebra on the fp16
    operands (one rounding at the end) and the reference's eager fp16 solve."""
    from pararnn_amd import fused_newton, newton_apply

    monkeypatch.setenv("PRNN_GRU_REPLAY_MFMA", mfma_replay)
    print(f"case gru_head_fp16 (mfma replay {mfma_replay})", flush=True)
    t, m = load_golden("gru_head_fp16")
    cell = _gru_cell(t, m)
    h0 = t["h0"].to(DEV)
    p = O.GRUHeadParams(t["W"], t["b"], t["A_z"], t["A_r"], t["A_n"])
    with torch.no_grad():
        out = fused_newton(cell, t["wx"].to(DEV), max_iters=m["K"], omega=1.0,
                           h0=h0).float().cpu()
        out2 = newton_apply(cell, t["x"].to(DEV), _cfg(m["K"]), h0=h0).float().cpu()
    ref = O.gru_head_newton(p, None, max_iters=m["K"], wx=t["wx"], h0=t["h0"],
                            work="fused").float()
    eager = t["newton"].float()
    rel = ((out - ref).abs().max() / ref.abs().max()).item()
    rel_e = ((out - eager).abs().max() / eager.abs().max()).item()
    print(f"  rel vs fused semantics {rel:.2e}, vs reference eager fp16 {rel_e:.2e}", flush=True)
    # Phi is composed from bf16-rounded operands (the carry between chunks)
    assert rel <= 5e-3 and rel_e <= 5e-3
    assert ((out2 - out).abs().max() / out.abs().max()).item() <= 2e-3


def test_gru_head_backward_op_vs_float64():
    from oracle.backward import gru_head_backward

    from pararnn_amd import ops

    print("case gru_head_bwd_fp16 op vs float64", flush=True)
    t, m = load_golden("gru_head_bwd_fp16")
    p = O.GRUHeadParams(t["W"], t["b"], t["A_z"], t["A_r"], t["A_n"])
    wx = p.wx(t["x"])
    g_wx, g_a, _ = ops.gru_head_backward_fused(wx.to(DEV), *(a.to(DEV) for a in p.mats()), None,
                                               t["newton"].to(DEV), t["grad"].to(DEV))
    p64 = O.GRUHeadParams(*(v.double() for v in (p.W, p.b, p.A_z, p.A_r, p.A_n)))
    ex = gru_head_backward(p64, t["x"].double(), t["newton"].double(), t["grad"].double(),
                           work=torch.float64, wx=wx.double())

    def rel(a, b):
        a, b = a.double().cpu(), b.double().cpu()
        return ((a - b).abs().max() / b.abs().max()).item()

    errs = {"g_wx": rel(g_wx, ex["g_wx"])}
    for i, k in enumerate(("A_z", "A_r", "A_n")):
        errs[k] = rel(g_a[i], ex[k])
    print("  rel err " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    assert g_wx.dtype == F16
    # g_A is contracted from the gate gradients as stored (g_wx, rounded to
    # fp16: 2^-11 relative per element), so it carries that rounding too
    assert errs["g_wx"] <= 1e-3 and max(errs[k] for k in ("A_z", "A_r", "A_n")) <= 1e-3


@pytest.mark.parametrize("case", ["mixed", "tiny"])
def test_packed_stream_vs_each_sequence_alone(case):
    """fp16 packed stream (carry cut at each head in-kernel) against the
    rectangular kernels run on each sequence alone."""
    from pararnn_amd import ParaSLSTM, ops

    lengths = {"mixed": [1, 5, 37, 300, 2, 1, 64, 1000, 3, 129],
               "tiny": [1] * 7 + [2] * 5 + [3] * 4}[case]
    print(f"case packed fp16 {case}", flush=True)
    torch.manual_seed(21)
    cell = ParaSLSTM(9, 128).to(DEV, F16)
    g = torch.Generator().manual_seed(22)
    x = torch.randn(1, sum(lengths), 9, generator=g).to(DEV, F16)
    h0 = torch.randn(len(lengths), 4, 128, generator=g) * 0.5
    h0[:, 1] = h0[:, 1].abs() + 0.5
    h0 = h0.to(DEV, F16)
    cs = torch.tensor([0] + lengths).cumsum(0).to(DEV)
    with torch.no_grad():
        wx = cell.W_x(x)
        r = cell.clipped_r()
        init = ops.slstm_init_fused(wx, r, h0, cs, picard_iters=3, eps=cell.eps)
        out = ops.newton_slstm_fused(wx, r, h0, init, None, cs, max_iters=2, omega=1.0,
                                     eps=cell.eps)
        inits, outs = [], []
        for s, (a, b) in enumerate(zip(cs[:-1].tolist(), cs[1:].tolist())):
            w = wx[:, a:b].contiguous()
            i1 = ops.slstm_init_fused(w, r, h0[s:s + 1], picard_iters=3, eps=cell.eps)
            inits.append(i1)
            outs.append(ops.newton_slstm_fused(w, r, h0[s:s + 1], i1, max_iters=2, omega=1.0,
                                               eps=cell.eps))
    ref_init, ref = torch.cat(inits, 1).float(), torch.cat(outs, 1).float()
    n_init = ((init.float() - ref_init).norm() / ref_init.norm()).item()
    n_out = ((out.float() - ref).norm() / ref.norm()).item()
    print(f"  norm-rel init {n_init:.2e}  newton {n_out:.2e}", flush=True)
    assert n_init <= 2e-4 and n_out <= 2e-3
