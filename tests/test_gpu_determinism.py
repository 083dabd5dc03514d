"""Run-to-run determinism on the GPU (the reference's bit-match of the packed
VJP, pararnn/determinism.py:77-113, widened to the whole fused path).

With ``torch.use_deterministic_algorithms(True)`` the sLSTM look-back scans run
in their deterministic mode: two identical forward + backward passes must
agree bit for bit, and the one-shot VJP re-run check must stay silent.  Its
states agree with the default mode's to 1e-5 (the golden parity tests run in
both modes).  The head GRU scans are deterministic in either mode.  Shapes are
large enough (hundreds of tiles per launch) that the default look-back's
timing-dependent walks do occur."""

import logging

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture
def deterministic():
    from pararnn_amd import determinism

    prev = torch.are_deterministic_algorithms_enabled()
    prev_warn = torch.is_deterministic_algorithms_warn_only_enabled()
    torch.use_deterministic_algorithms(True, warn_only=True)
    determinism.reset_checks()
    yield
    torch.use_deterministic_algorithms(prev, warn_only=prev_warn)
    determinism.reset_checks()


def _cfg(K=2, P=5):
    from pararnn_amd import NewtonConfig

    return NewtonConfig(max_iters=K, picard_iters=P, residual_atol=None, residual_fail=None,
                        picard_adapt=False, scan_backend="fused")


def _slstm(dtype, d_in=128, d=256, seed=0):
    from pararnn_amd import ParaSLSTM

    torch.manual_seed(seed)
    return ParaSLSTM(d_in, d, mix="diag").to(device=DEV, dtype=dtype)


def _run(cell, x, h0, grad, cfg):
    """One forward + backward; returns states and every gradient (cloned)."""
    from pararnn_amd import newton_apply

    cell.zero_grad(set_to_none=True)
    xx = x.clone().requires_grad_(True)
    hh = None if h0 is None else h0.clone().requires_grad_(True)
    H = newton_apply(cell, xx, cfg, h0=hh)
    (H.float() * grad).sum().backward()
    out = {"H": H.detach().clone(), "x": xx.grad.clone()}
    if hh is not None:
        out["h0"] = hh.grad.clone()
    for n, p in cell.named_parameters():
        out[n] = p.grad.clone()
    torch.cuda.synchronize()
    return out


def _bitequal(a, b):
    return {k: bool(torch.equal(a[k].view(torch.uint8), b[k].view(torch.uint8))) for k in a}


def _inputs(cell, B, T, dtype, seed=1, h0_slots=4):
    g = torch.Generator().manual_seed(seed)
    d_in, d = cell.W_x.in_features, cell.R.shape[-1] if hasattr(cell, "R") else None
    x = torch.randn(B, T, d_in, generator=g).to(DEV, dtype)
    grad = torch.randn(B, T, h0_slots, d, generator=g).to(DEV)
    h0 = (0.1 * torch.randn(B, h0_slots, d, generator=g)).to(DEV, dtype)
    return x, h0, grad


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_slstm_deterministic_bitmatch(deterministic, dtype, caplog):
    B, T = 2, 8192
    print(f"case determinism sLSTM diag {dtype} B={B} T={T} d=256", flush=True)
    cell = _slstm(dtype)
    x, h0, grad = _inputs(cell, B, T, dtype)
    with caplog.at_level(logging.WARNING, logger="pararnn_amd"):
        a = _run(cell, x, h0, grad, _cfg())
        b = _run(cell, x, h0, grad, _cfg())
    from pararnn_amd import _lib

    assert _lib.load().prnn_deterministic() == 1
    eq = _bitequal(a, b)
    print(f"  bit-equal: {eq}", flush=True)
    assert all(eq.values()), eq
    assert not [r for r in caplog.records if "differed" in r.getMessage()]
    assert all(torch.isfinite(v.float()).all() for v in a.values())


def test_slstm_deterministic_mode_matches_default():
    """The deterministic walk changes only the grouping of the carry
    arithmetic: the fp32 states agree with the default mode to 1e-5 relative.
    (Gradients are checked against the oracle in both modes by the sLSTM
    backward tests; between the two modes they move by the backward scan's
    own sensitivity to last-bit differences of the states, ~1e-4 here.)"""
    from pararnn_amd import _lib

    B, T = 2, 8192
    print(f"case determinism sLSTM fp32 deterministic vs default mode B={B} T={T}", flush=True)
    cell = _slstm(torch.float32)
    x, h0, grad = _inputs(cell, B, T, torch.float32)
    prev = torch.are_deterministic_algorithms_enabled()
    try:
        torch.use_deterministic_algorithms(False)
        a = _run(cell, x, h0, grad, _cfg())
        assert _lib.load().prnn_deterministic() == 0
        torch.use_deterministic_algorithms(True, warn_only=True)
        b = _run(cell, x, h0, grad, _cfg())
        assert _lib.load().prnn_deterministic() == 1
    finally:
        torch.use_deterministic_algorithms(prev)
    for k in a:
        ref = a[k].double()
        rel = ((b[k].double() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
        print(f"  {k}: rel {rel:.2e}", flush=True)
        assert rel <= (1e-5 if k == "H" else 1e-3), k


def test_slstm_ops_deterministic_repeat(deterministic):
    """The three sLSTM launches through the ops layer, several repeats, bf16
    at a longer shape (more tiles in flight, more look-back variety)."""
    from pararnn_amd import ops

    B, T, d = 1, 32768, 512
    print(f"case determinism sLSTM ops bf16 B={B} T={T} d={d} x4", flush=True)
    g = torch.Generator().manual_seed(3)
    wx = (0.5 * torch.randn(B, T, 4 * d, generator=g)).to(DEV, torch.bfloat16)
    r = (0.3 * torch.rand(4, d, generator=g) - 0.15).to(DEV, torch.bfloat16)
    grad = torch.randn(B, T, 4, d, generator=g).to(DEV, torch.bfloat16)
    # a packed stream of the same tokens (several sequences) and K = 1, which
    # also takes the single fused launch
    cs = torch.tensor([0, 5000, 5001, 17000, 32768], device=DEV)
    outs = []
    for _ in range(4):
        guess = ops.slstm_init_fused(wx, r, None, picard_iters=5, eps=1e-6)
        H = ops.newton_slstm_fused(wx, r, None, guess, max_iters=2, omega=1.0, eps=1e-6)
        H1 = ops.newton_slstm_fused(wx, r, None, guess, max_iters=1, omega=1.0, eps=1e-6)
        g_wx, g_r, g_h0, g_b = ops.slstm_backward_fused(wx, r, None, H, grad, eps=1e-6)
        pg = ops.slstm_init_fused(wx, r, None, cs, picard_iters=5, eps=1e-6)
        pH = ops.newton_slstm_fused(wx, r, None, pg, None, cs, max_iters=2, omega=1.0, eps=1e-6)
        pH1 = ops.newton_slstm_fused(wx, r, None, pg, None, cs, max_iters=1, omega=1.0, eps=1e-6)
        torch.cuda.synchronize()
        outs.append({"guess": guess, "H": H, "H1": H1, "g_wx": g_wx, "g_r": g_r, "g_b": g_b,
                     "packed_guess": pg, "packed_H": pH, "packed_H1": pH1})
    for o in outs[1:]:
        eq = _bitequal(outs[0], o)
        assert all(eq.values()), eq


def test_gru_head_bitmatch_default_mode():
    """The head GRU's carry scan and reductions run in a fixed order: two
    identical passes agree bit for bit without the deterministic flag."""
    from pararnn_amd import ParaGRU

    B, T, H = 2, 4096, 4
    print(f"case determinism GRU head fp32 B={B} T={T} H={H}", flush=True)
    torch.manual_seed(0)
    cell = ParaGRU(64, 64 * H, mix="head", n_heads=H).to(DEV)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(B, T, 64, generator=g).to(DEV)
    grad = torch.randn(B, T, 64 * H, generator=g).to(DEV)
    h0 = (0.1 * torch.randn(B, 64 * H, generator=g)).to(DEV)
    a = _run(cell, x, h0, grad, _cfg(K=3, P=0))
    b = _run(cell, x, h0, grad, _cfg(K=3, P=0))
    eq = _bitequal(a, b)
    print(f"  bit-equal: {eq}", flush=True)
    assert all(eq.values()), eq


def test_tagged_workspace_matches_cleared(monkeypatch):
    """The cached, tag-based sLSTM workspace gives bit-identical results to a
    fresh, cleared workspace per call (deterministic mode makes both exact),
    over a sequence of calls whose shapes grow and shrink, across a forced
    re-zero at the tag limit."""
    from pararnn_amd import ops

    prev = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True, warn_only=True)
    try:
        shapes = [(1, 4096, 256), (2, 8192, 128), (1, 2048, 512), (2, 8192, 128), (1, 4096, 256)]
        g = torch.Generator().manual_seed(5)
        cases = []
        for B, T, d in shapes:
            wx = (0.5 * torch.randn(B, T, 4 * d, generator=g)).to(DEV, torch.bfloat16)
            r = (0.3 * torch.rand(4, d, generator=g) - 0.15).to(DEV, torch.bfloat16)
            grad = torch.randn(B, T, 4, d, generator=g).to(DEV, torch.bfloat16)
            cases.append((wx, r, grad))

        def run_all():
            outs = []
            for wx, r, grad in cases:
                guess = ops.slstm_init_fused(wx, r, None, picard_iters=5, eps=1e-6)
                H = ops.newton_slstm_fused(wx, r, None, guess, max_iters=2, omega=1.0, eps=1e-6)
                g_wx, g_r, _, _ = ops.slstm_backward_fused(wx, r, None, H, grad, eps=1e-6)
                outs.append((guess, H, g_wx, g_r))
            torch.cuda.synchronize()
            return outs

        print("case tagged workspace vs cleared workspace (5 shapes x 3 ops)", flush=True)
        monkeypatch.setenv("PARARNN_AMD_TAGGED_WS", "0")
        ref = run_all()
        monkeypatch.setenv("PARARNN_AMD_TAGGED_WS", "1")
        ops.release_workspaces()
        got = run_all()
        got2 = run_all()  # the cached buffer, tags well past the first pass
        monkeypatch.setattr(ops, "_TAG_BASE_MAX", 64 * 7)  # forces re-zeroed buffers
        got3 = run_all()
        for a, b, c, e in zip(ref, got, got2, got3):
            for x, y, z, w in zip(a, b, c, e):
                assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))
                assert torch.equal(x.view(torch.uint8), z.view(torch.uint8))
                assert torch.equal(x.view(torch.uint8), w.view(torch.uint8))
    finally:
        torch.use_deterministic_algorithms(prev)
        ops.release_workspaces()
