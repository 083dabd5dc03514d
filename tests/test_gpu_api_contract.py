"""Contract checks of the drop-in boundary that the reference's (unshipped)
test suite names (test_noncontiguous, test_custom_ops, test_autocast,
test_compile, test_overflow_stress): outer autocast is switched off for the
solve (newton/__init__.py:193-209, 305), non-contiguous inputs give the same
results, the torch.library ops pass torch's op checks and trace under
torch.compile, and saturated / exponent-overflowing gate pre-activations stay
finite and match the oracle."""

import pytest
import torch

import oracle as O
from oracle.slstm import slstm_newton_f64

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _cfg(K=2, P=3):
    from pararnn_amd import NewtonConfig

    return NewtonConfig(max_iters=K, picard_iters=P, residual_atol=None, residual_fail=None,
                        picard_adapt=False)


@pytest.fixture
def deterministic():
    prev = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True, warn_only=True)
    yield
    torch.use_deterministic_algorithms(prev)


def _slstm_cell(d=128, d_in=32, seed=0):
    from pararnn_amd import ParaSLSTM

    torch.manual_seed(seed)
    return ParaSLSTM(d_in, d).to(DEV)


def _gru_cell(H=2, d_in=32, seed=0):
    from pararnn_amd import ParaGRU

    torch.manual_seed(seed)
    return ParaGRU(d_in, 64 * H, mix="head", n_heads=H).to(DEV)


def _fwd_bwd(cell, x, cfg):
    from pararnn_amd import newton_apply

    cell.zero_grad(set_to_none=True)
    xx = x.detach().clone().requires_grad_(True)
    H = newton_apply(cell, xx, cfg)
    H.float().square().sum().backward()
    return H.detach(), xx.grad, [p.grad for p in cell.parameters()]


@pytest.mark.parametrize("kind", ["slstm", "gru"])
def test_outer_autocast_is_switched_off(kind, deterministic):
    print(f"case autocast {kind}", flush=True)
    cell = _slstm_cell() if kind == "slstm" else _gru_cell()
    x = torch.randn(2, 3000, 32, device=DEV)
    cfg = _cfg() if kind == "slstm" else _cfg(K=3, P=0)
    ref = _fwd_bwd(cell, x, cfg)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        got = _fwd_bwd(cell, x, cfg)
    assert got[0].dtype == torch.float32
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
    for a, b in zip(got[2], ref[2]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("kind", ["slstm", "gru"])
def test_noncontiguous_inputs(kind, deterministic):
    from pararnn_amd import newton_apply, ops

    print(f"case noncontiguous {kind}", flush=True)
    cell = _slstm_cell() if kind == "slstm" else _gru_cell()
    big = torch.randn(2, 3000, 64, device=DEV)
    x = big[:, :, ::2]  # stride 2 in the feature dim
    assert not x.is_contiguous()
    cfg = _cfg() if kind == "slstm" else _cfg(K=3, P=0)
    with torch.no_grad():
        a = newton_apply(cell, x, cfg)
        b = newton_apply(cell, x.contiguous(), cfg)
        assert torch.equal(a, b)
        if kind == "slstm":
            d = cell.R.shape[-1]
            wide = torch.randn(2, 3000, 4 * d + 16, device=DEV)
            wx = wide[..., :4 * d]  # a view with a padded row stride
            r = cell.clipped_r()
            r_t = r.t().contiguous().t()  # same values, transposed strides
            g = ops.slstm_init_fused(wx, r_t, None, picard_iters=3, eps=cell.eps)
            assert torch.equal(g, ops.slstm_init_fused(wx.contiguous(), r, None, picard_iters=3,
                                                       eps=cell.eps))
            gpad = torch.zeros(*g.shape[:-1], d + 8, device=DEV)
            gpad[..., :d] = g
            h = ops.newton_slstm_fused(wx, r_t, None, gpad[..., :d], max_iters=2, omega=1.0,
                                       eps=cell.eps)
            assert torch.equal(h, ops.newton_slstm_fused(wx.contiguous(), r, None, g,
                                                         max_iters=2, omega=1.0, eps=cell.eps))


def test_opcheck_schema_and_fake():
    from pararnn_amd import ops

    print("case torch.library.opcheck", flush=True)
    d = 64
    wx = torch.randn(2, 100, 4 * d, device=DEV)
    r = torch.rand(4, d, device=DEV) - 0.5
    guess = ops.slstm_init_fused(wx, r, None, picard_iters=2, eps=1e-6)
    util = ("test_schema", "test_faketensor")
    torch.library.opcheck(torch.ops.pararnn.slstm_init_fused.default, (wx, r, None),
                          {"picard_iters": 2, "eps": 1e-6}, test_utils=util)
    torch.library.opcheck(torch.ops.pararnn.newton_slstm_fused.default, (wx, r, None, guess),
                          {"max_iters": 2, "omega": 1.0, "eps": 1e-6}, test_utils=util)
    torch.library.opcheck(torch.ops.pararnn.slstm_backward_fused.default,
                          (wx, r, None, guess, torch.randn_like(guess)), {"eps": 1e-6},
                          test_utils=util)
    H = 2
    wg = torch.randn(2, 100, 3 * 64 * H, device=DEV)
    a = [torch.randn(H, 64, 64, device=DEV) * 0.1 for _ in range(3)]
    torch.library.opcheck(torch.ops.pararnn.newton_gru_head_fused.default, (wg, *a, None),
                          {"max_iters": 2, "omega": 1.0}, test_utils=util)
    out = ops.newton_gru_head_fused(wg, *a, None, max_iters=2, omega=1.0)
    torch.library.opcheck(torch.ops.pararnn.gru_head_backward_fused.default,
                          (wg, *a, None, out, torch.randn_like(out)), test_utils=util)


def test_torch_compile_traces_the_ops(deterministic):
    from pararnn_amd import newton_apply

    print("case torch.compile(aot_eager)", flush=True)
    cell = _slstm_cell()
    x = torch.randn(2, 2000, 32, device=DEV)
    cfg = _cfg()

    def f(x):
        return newton_apply(cell, x, cfg)

    with torch.no_grad():
        ref = f(x)
        got = torch.compile(f, backend="aot_eager")(x)
    assert torch.equal(got, ref)


def test_overflowing_gate_exponents_slstm():
    """Input and forget pre-activations of |z| ~ 300 (e^300 overflows fp32):
    the max-stabilised cell stays finite and matches the oracle."""
    from pararnn_amd import ParaSLSTM, newton_apply

    print("case overflow stress sLSTM", flush=True)
    torch.manual_seed(11)
    d = 64
    cell = ParaSLSTM(7, d)
    with torch.no_grad():
        cell.W_x.weight[:2 * d] *= 80.0
    x = torch.randn(2, 400, 7)
    p = O.SLSTMParams(cell.W_x.weight.detach(), cell.W_x.bias.detach(), cell.R.detach())
    assert p.wx(x)[..., :2 * d].abs().max() > 200
    with torch.no_grad():
        ref = O.slstm_newton(p, x, max_iters=2, picard_iters=3)
        _, exact = slstm_newton_f64(p, p.wx(x), max_iters=2, picard_iters=3)
        out = newton_apply(cell.to(DEV), x.to(DEV), _cfg(2, 3))
    assert torch.isfinite(out).all()
    # fp32 rounding grows with |m| ~ 1e2..1e4 here, for the reference's own
    # algorithm too: the bar is the reference's fp32 distance to float64.
    got, ref, exact = out.double().cpu(), ref.double(), exact.double()
    e_ours = ((got - exact).abs() / (1 + exact.abs())).amax(dim=(0, 1, 3))
    e_ref = ((ref - exact).abs() / (1 + exact.abs())).amax(dim=(0, 1, 3))
    print(f"  per slot (c,n,m,h) rel to float64: gpu {e_ours.tolist()} reference {e_ref.tolist()}",
          flush=True)
    assert torch.all(e_ours <= torch.clamp(1.5 * e_ref, min=3e-5))


def test_saturated_gates_gru_head():
    from pararnn_amd import ParaGRU, newton_apply

    print("case overflow stress GRU head", flush=True)
    torch.manual_seed(12)
    cell = ParaGRU(10, 128, mix="head", n_heads=2)
    x = torch.randn(2, 300, 10) * 60.0
    p = O.GRUHeadParams(cell.W_x.weight.detach(), cell.W_x.bias.detach(), cell.A_z.detach(),
                        cell.A_r.detach(), cell.A_n.detach())
    with torch.no_grad():
        ref = O.gru_head_newton(p, x, max_iters=3)
        out = newton_apply(cell.to(DEV), x.to(DEV), _cfg(3, 0)).cpu()
    assert torch.isfinite(out).all()
    err = (out - ref).abs().max().item()
    print(f"  max|gpu-oracle| {err:.2e}", flush=True)
    assert err <= 1e-5
