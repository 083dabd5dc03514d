"""Host-side API: config validation, dispatch and error behaviour (CPU only)."""

import pytest
import torch

from pararnn_amd import (
    NewtonConfig,
    ParaGRU,
    ParaSLSTM,
    compile_safe_config,
    newton_apply,
    slstm_auto_picard,
    slstm_picard_next,
)
from pararnn_amd.config import lookup_iters_by_t, validate_config


def test_defaults_match_reference():
    c = NewtonConfig()
    assert (c.max_iters, c.omega, c.scan_backend, c.residual_atol, c.residual_fail) == (
        3, 1.0, "auto", 1e-5, 1.0)
    assert c.picard_iters is None and c.picard_adapt is None and c.scan_tile == "assoc"
    s = compile_safe_config(scan_backend="fused")
    assert s.residual_atol is None and s.residual_fail is None and s.picard_adapt is False


@pytest.mark.parametrize("kw", [
    dict(scan_backend="bogus"), dict(max_iters=-1), dict(picard_iters=-2),
    dict(scan_tile="x"), dict(fused_window_len=64), dict(coords="x"),
    dict(newton_iters_by_t={64: 2}), dict(residual_fail=-1.0),
])
def test_invalid_configs_raise(kw):
    with pytest.raises(ValueError):
        validate_config(NewtonConfig(**kw))


def test_picard_ladder_and_k_schedule():
    assert [slstm_auto_picard(t) for t in (1, 64, 65, 2048, 2049)] == [1, 1, 3, 3, 5]
    assert [slstm_picard_next(p) for p in (0, 1, 3, 5)] == [1, 3, 5, None]
    assert lookup_iters_by_t({64: 2, 1024: 3, 4096: 4}, 1000) == 2
    assert lookup_iters_by_t({64: 2, 1024: 3, 4096: 4}, 10) == 2
    assert lookup_iters_by_t({64: 2, 1024: 3, 4096: 4}, 5000) == 4


def test_weights_match_reference_init():
    from conftest import load_golden

    t, m = load_golden("slstm_cfg1_fp32")
    torch.manual_seed(m["seed"])
    cell = ParaSLSTM(m["d_in"], m["d"], mix="diag")
    assert torch.equal(cell.W_x.weight, t["W"]) and torch.equal(cell.R, t["R"])
    t, m = load_golden("gru_head_fp32")
    torch.manual_seed(m["seed"])
    g = ParaGRU(m["d_in"], m["n_heads"] * m["d_head"], mix="head", n_heads=m["n_heads"])
    assert torch.equal(g.A_z, t["A_z"]) and torch.equal(g.A_n, t["A_n"])


def test_cell_step_matches_oracle():
    import oracle as O
    from conftest import load_golden

    t, _ = load_golden("parts")
    cell = ParaSLSTM(8, 16)
    with torch.no_grad():
        cell.R.copy_(t["slstm_R"])
        new, jac = cell.step_with_jacobian(t["slstm_state"], None, wx=t["slstm_wx"])
    assert torch.equal(new, t["slstm_new"]) and torch.equal(jac, t["slstm_jac"])
    g = ParaGRU(8, 128, mix="head", n_heads=2)
    with torch.no_grad():
        for k in ("A_z", "A_r", "A_n"):
            getattr(g, k).copy_(t["gru_" + k])
        gnew, gjac = g.step_with_jacobian(t["gru_h"], None, wx=t["gru_wx"])
    assert torch.equal(gnew, t["gru_new"]) and torch.equal(gjac, t["gru_jac"])
    del O


def test_cpu_input_fails_loudly():
    cell = ParaSLSTM(4, 8)
    x = torch.randn(1, 5, 4)
    with torch.no_grad():
        with pytest.raises(TypeError, match="ROCm GPU"):
            newton_apply(cell, x, NewtonConfig(scan_backend="fused"))
        with pytest.raises(TypeError, match="ROCm GPU"):
            newton_apply(cell, x)
        # the eager loop runs on the GPU too: a CPU tensor is refused, not
        # solved by torch ops
        with pytest.raises(TypeError, match="ROCm GPU"):
            newton_apply(cell, x, NewtonConfig(scan_backend="eager"))
        with pytest.raises(NotImplementedError):
            newton_apply(cell, x, NewtonConfig(scan_backend="triton"))


def test_unsupported_cells_and_knobs():
    with pytest.raises(NotImplementedError):
        ParaSLSTM(4, 8, mix="head", n_heads=2)
    with pytest.raises(ValueError):
        ParaGRU(4, 8, mix="head", n_heads=3)
    with pytest.raises(TypeError):
        newton_apply(ParaGRU(4, 8), torch.randn(1, 3, 4), NewtonConfig(picard_iters=2))


def test_grad_mode_on_cpu_input_fails_loudly():
    cell = ParaSLSTM(4, 8)
    with pytest.raises(TypeError, match="ROCm GPU"):
        newton_apply(cell, torch.randn(1, 5, 4))


def test_ops_validate_before_launch():
    from pararnn_amd import ops

    wx = torch.randn(1, 4, 16)
    with pytest.raises(ValueError):
        ops.newton_slstm_fused(wx, torch.randn(4, 5), max_iters=1, omega=1.0, eps=1e-6)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.newton_slstm_fused(wx, torch.randn(4, 4), max_iters=1, omega=1.0, eps=1e-6)
    with pytest.raises(TypeError):
        ops.newton_slstm_fused(wx, torch.randn(4, 4), max_iters=1, omega=1.0, eps=1e-6,
                               log_coords=True)
    a = torch.randn(2, 64, 64)
    with pytest.raises(ValueError):
        ops.newton_gru_head_fused(torch.randn(1, 3, 100), a, a, a, max_iters=1, omega=1.0)


def test_decode_step_host_rules():
    # CPU tensors: the reference runs the cell's own step there
    # (kernels/decode.py:172-179); block_table needs the GPU kernel.
    from pararnn_amd import ParaSLSTM, can_decode_step, decode_step, decode_wx

    torch.manual_seed(0)
    cell = ParaSLSTM(6, 8)
    state = torch.zeros(2, 4, 8)
    x = torch.randn(2, 1, 6)
    assert not can_decode_step(cell, x)
    with torch.no_grad():
        y = decode_step(cell, state, x[:, 0])
        assert torch.allclose(y, cell.step(state, x[:, 0]))
        assert decode_wx(cell, x).shape == (2, 32)
        with pytest.raises(RuntimeError, match="block_table"):
            decode_step(cell, state, x[:, 0], block_table=torch.tensor([0, 1]))
    with pytest.raises(ValueError, match="x or wx"):
        decode_step(cell, state)
