"""Pin the CPU oracle: golden vectors from the reference plus checks the
mathematics fixes (autograd Jacobians, brute-force scans, Newton's fixed
point, the R = 0 special case).  CPU only."""

import pytest
import torch
from conftest import load_golden

import oracle as O
from oracle.slstm import prepend

SLSTM_CASES = [
    "slstm_cfg1_fp32", "slstm_h0_fp32", "slstm_bf16", "slstm_fp16", "slstm_long_fp32"]
GRU_CASES = ["gru_head_fp32", "gru_head_h0_fp32", "gru_head_bf16", "gru_head_fp16"]


def _slstm_params(t):
    return O.SLSTMParams(t["W"], t["b"], t["R"])


def _gru_params(t):
    return O.GRUHeadParams(t["W"], t["b"], t["A_z"], t["A_r"], t["A_n"])


@pytest.mark.parametrize("name", SLSTM_CASES)
def test_slstm_oracle_matches_reference_bitwise(name):
    t, m = load_golden(name)
    p = _slstm_params(t)
    wx = t["wx"] if "wx" in t else p.wx(t["x"])
    h0 = t.get("h0")
    assert torch.equal(O.picard_init(p, wx, m["P"], h0), t["init"])
    out = O.slstm_newton(p, t["x"], max_iters=m["K"], picard_iters=m["P"], h0=h0, wx=wx)
    assert torch.equal(out, t["newton"])
    assert torch.equal(O.slstm_sequential(p, t["x"], h0, wx=wx), t["sequential"])


@pytest.mark.parametrize("name", GRU_CASES)
def test_gru_head_oracle_matches_reference_bitwise(name):
    t, m = load_golden(name)
    p = _gru_params(t)
    h0 = t.get("h0")
    out = O.gru_head_newton(p, t["x"], max_iters=m["K"], h0=h0, wx=t["wx"])
    assert torch.equal(out, t["newton"])
    assert torch.equal(O.gru_head_sequential(p, t["x"], h0, wx=t["wx"]), t["sequential"])


def test_parts_match_reference():
    t, _ = load_golden("parts")
    p = O.SLSTMParams(torch.zeros(64, 8), torch.zeros(64), t["slstm_R"])
    new, jac = O.slstm_jacobian(p, t["slstm_state"], t["slstm_wx"])
    assert torch.equal(new, t["slstm_new"]) and torch.equal(jac, t["slstm_jac"])
    assert torch.equal(O.scan_block4(t["scan4_j"], t["scan4_r"]), t["scan4_out"])
    assert torch.equal(O.scan_dense(t["scand_j"], t["scand_r"]), t["scand_out"])
    assert torch.equal(O.frozen_gate_scan(t["fg_pre"], 1e-6, t["fg_h0"]), t["fg_out"])
    assert torch.equal(O.frozen_gate_scan(t["fg_pre"], 1e-6, None), t["fg_out_noh0"])
    g = O.GRUHeadParams(torch.zeros(384, 8), torch.zeros(384), t["gru_A_z"], t["gru_A_r"],
                        t["gru_A_n"])
    gnew, gjac = O.gru_head_jacobian(g, t["gru_h"], t["gru_wx"])
    assert torch.equal(gnew, t["gru_new"]) and torch.equal(gjac, t["gru_jac"])


def test_slstm_jacobian_matches_autograd_float64():
    g = torch.Generator().manual_seed(0)
    d = 6
    p = O.SLSTMParams(torch.zeros(4 * d, 3, dtype=torch.float64),
                      torch.zeros(4 * d, dtype=torch.float64),
                      torch.randn(4, d, generator=g, dtype=torch.float64) * 0.4)
    prev = torch.randn(4, d, generator=g, dtype=torch.float64)
    prev[1] = prev[1].abs() + 0.5
    wx = torch.randn(4 * d, generator=g, dtype=torch.float64)
    _, jac = O.slstm_jacobian(p, prev, wx)
    full = torch.autograd.functional.jacobian(lambda s: O.slstm_step(p, s, wx), prev)
    # full[o, ch, i, ch2] is zero off the channel diagonal; jac is [o, i, ch]
    for ch in range(d):
        torch.testing.assert_close(jac[:, :, ch], full[:, ch, :, ch], rtol=1e-10, atol=1e-12)
    off = full.clone()
    for ch in range(d):
        off[:, ch, :, ch] = 0
    assert off.abs().max() == 0


def test_gru_head_jacobian_matches_autograd_float64():
    g = torch.Generator().manual_seed(1)
    hh, dh = 2, 5
    mk = lambda: torch.randn(hh, dh, dh, generator=g, dtype=torch.float64) * 0.3  # noqa: E731
    p = O.GRUHeadParams(torch.zeros(3 * hh * dh, 2, dtype=torch.float64),
                        torch.zeros(3 * hh * dh, dtype=torch.float64), mk(), mk(), mk())
    h = torch.randn(hh * dh, generator=g, dtype=torch.float64)
    wx = torch.randn(3 * hh * dh, generator=g, dtype=torch.float64)
    _, jac = O.gru_head_jacobian(p, h, wx)
    full = torch.autograd.functional.jacobian(lambda v: O.gru_head_step(p, v, wx), h)
    for k in range(hh):
        sl = slice(k * dh, (k + 1) * dh)
        torch.testing.assert_close(jac[k], full[sl, sl], rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("kind,shape_j,shape_r", [
    ("block4", (2, 37, 4, 4, 3), (2, 37, 4, 3)),
    ("dense", (3, 19, 5, 5), (3, 19, 5)),
    ("diag", (2, 33, 4), (2, 33, 4)),
    ("block4", (1, 1, 4, 4, 2), (1, 1, 4, 2)),
])
def test_blelloch_equals_sequential_recurrence(kind, shape_j, shape_r):
    g = torch.Generator().manual_seed(3)
    j = torch.randn(*shape_j, generator=g, dtype=torch.float64) * 0.5
    r = torch.randn(*shape_r, generator=g, dtype=torch.float64)
    torch.testing.assert_close(O.blelloch_inclusive(j, r, kind), O.sequential_affine(j, r, kind),
                               rtol=1e-10, atol=1e-10)


def test_zero_jacobian_scan_is_identity():
    r = torch.randn(2, 10, 4, 3, dtype=torch.float64)
    assert torch.equal(O.scan_block4(torch.zeros(2, 10, 4, 4, 3, dtype=torch.float64), r), r)


def test_frozen_gate_is_exact_when_r_is_zero():
    # R = 0: the cell has no h-coupling, so the frozen-gate scan is the solution
    # and one Newton step leaves the residual at rounding level.  The scan works
    # in fp32 internally (as the reference's does), hence fp32 tolerances.
    g = torch.Generator().manual_seed(4)
    d, T = 5, 60
    p = O.SLSTMParams(torch.zeros(4 * d, 3, dtype=torch.float64),
                      torch.zeros(4 * d, dtype=torch.float64),
                      torch.zeros(4, d, dtype=torch.float64))
    wx = torch.randn(2, T, 4 * d, generator=g, dtype=torch.float64) * 2
    seq = O.slstm_sequential(p, None, wx=wx)
    init = O.frozen_gate_scan(wx, p.eps)
    torch.testing.assert_close(init, seq, rtol=2e-6, atol=2e-6)
    pred = O.slstm_step(p, prepend(init, None), wx)
    assert (pred - init).abs().max() < 2e-5


def test_max_plus_stabiliser_matches_brute_force():
    g = torch.Generator().manual_seed(5)
    pre = torch.randn(1, 50, 8, generator=g, dtype=torch.float64) * 3
    out = O.frozen_gate_scan(pre, 1e-6)
    zi, zf = pre[..., 0:2], pre[..., 2:4]
    m = torch.zeros(1, 2, dtype=torch.float64)
    for t in range(50):
        m = torch.maximum(zf[:, t] + m, zi[:, t])
        torch.testing.assert_close(out[:, t, 2], m, rtol=1e-5, atol=2e-5)  # fp32 inside


@pytest.mark.parametrize("name", ["slstm_h0_fp32", "gru_head_fp32"])
def test_newton_converges_to_sequential_in_float64(name):
    t, m = load_golden(name)
    if "R" in t:
        p = O.SLSTMParams(t["W"].double(), t["b"].double(), t["R"].double())
        h0 = t["h0"].double() if "h0" in t else None
        x = t["x"].double()
        out = O.slstm_newton(p, x, max_iters=8, picard_iters=m["P"], h0=h0)
        seq = O.slstm_sequential(p, x, h0)
    else:
        p = O.GRUHeadParams(*(t[k].double() for k in ("W", "b", "A_z", "A_r", "A_n")))
        x = t["x"].double()
        out = O.gru_head_newton(p, x, max_iters=6)
        seq = O.gru_head_sequential(p, x)
    assert (out - seq).abs().max() < 1e-9


def test_auto_picard_table():
    import json
    import os

    from conftest import GOLDEN

    table = json.load(open(os.path.join(GOLDEN, "auto_picard.json")))
    for t, p in table.items():
        assert O.auto_picard(int(t)) == p


def test_fused_semantics_is_closer_to_fp32_truth_than_bf16_eager():
    # Documents why bf16 parity is stated against the fused-op semantics.
    t, m = load_golden("slstm_bf16")
    p = _slstm_params(t)
    fused = O.slstm_newton(p, None, max_iters=m["K"], picard_iters=m["P"], wx=t["wx"],
                           work="fused").float()
    p32 = O.SLSTMParams(t["W"].float(), t["b"].float(), t["R"].float())
    truth = O.slstm_sequential(p32, None, wx=t["wx"].float())
    eager = t["newton"].float()
    err_f = ((fused - truth).norm() / truth.norm()).item()
    err_e = ((eager - truth).norm() / truth.norm()).item()
    assert err_f < 5e-3 and err_e > 3 * err_f
