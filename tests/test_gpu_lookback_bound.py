"""Bounded waits of the sLSTM look-back: with the polling budget cut to one
round (prnn_set_spin_limit), waves that would wait longer give up, every
kernel still ends, the call's status word reports it and, with
PARARNN_AMD_CHECK_STATUS=1, the op raises RuntimeError.  Afterwards the
default budget gives correct, finite results again.  The condition is forced
from the host through the library's own bounded wait; no kernel faults."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _case():
    from pararnn_amd import ParaSLSTM

    torch.manual_seed(0)
    cell = ParaSLSTM(64, 64).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(1)
    # one channel block, 1000+ chunks in one chain: many waits per launch
    x = torch.randn(1, 65536, 64, generator=g, device=DEV) * 0.5
    return cell, x


def test_give_up_is_reported_and_kernels_end(monkeypatch):
    from pararnn_amd import _lib, fused_newton

    lib = _lib.load()
    cell, x = _case()
    print("case look-back give-up: spin limit 1, T=65536, d=64", flush=True)
    det = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True, warn_only=True)
    try:
        with torch.no_grad():
            wx = cell.W_x(x)
            ref = fused_newton(cell, wx, max_iters=2, omega=1.0, h0=None, picard_iters=3)
    finally:
        torch.use_deterministic_algorithms(det)
    assert torch.isfinite(ref).all()
    monkeypatch.setenv("PARARNN_AMD_CHECK_STATUS", "1")
    raised = 0
    lib.prnn_set_spin_limit(1)
    try:
        for _ in range(4):
            try:
                with torch.no_grad():
                    fused_newton(cell, wx, max_iters=2, omega=1.0, h0=None, picard_iters=3)
            except RuntimeError as e:
                assert "gave up" in str(e)
                raised += 1
    finally:
        lib.prnn_set_spin_limit(0)
    torch.cuda.synchronize()
    print(f"  launches that reported a give-up: {raised} of 4", flush=True)
    assert raised >= 1
    # default budget: the same call (deterministic walk) is bit-equal to the
    # first solve
    torch.use_deterministic_algorithms(True, warn_only=True)
    try:
        with torch.no_grad():
            again = fused_newton(cell, wx, max_iters=2, omega=1.0, h0=None, picard_iters=3)
    finally:
        torch.use_deterministic_algorithms(det)
    print("  after restoring the budget: bit-equal to the first solve "
          f"{torch.equal(again, ref)}", flush=True)
    assert torch.equal(again, ref)


def test_wide_head_one_launch_give_up(monkeypatch):
    """The one-launch wide-head Newton solve waits for the previous iteration's
    tagged words; with a one-round budget the waiting walks give up, the
    launch ends, the status word reports it, and afterwards the default
    budget reproduces the first solve bit for bit."""
    from pararnn_amd import NewtonConfig, ParaGRU, _lib, newton_apply

    lib = _lib.load()
    torch.manual_seed(0)
    cell = ParaGRU(16, 256, mix="head", n_heads=2).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(2)
    x = torch.randn(2, 3000, 16, generator=g, device=DEV)
    cfg = NewtonConfig(max_iters=3, residual_atol=None, residual_fail=None)
    print("case wide one-launch give-up: spin limit 1, B=2, T=3000, d_head=128, K=3", flush=True)
    with torch.no_grad():
        ref = newton_apply(cell, x, cfg)
    assert torch.isfinite(ref).all()
    monkeypatch.setenv("PARARNN_AMD_CHECK_STATUS", "1")
    raised = 0
    lib.prnn_set_spin_limit(1)
    try:
        for _ in range(4):
            try:
                with torch.no_grad():
                    newton_apply(cell, x, cfg)
            except RuntimeError as e:
                assert "gave up" in str(e)
                raised += 1
    finally:
        lib.prnn_set_spin_limit(0)
    torch.cuda.synchronize()
    print(f"  launches that reported a give-up: {raised} of 4", flush=True)
    assert raised >= 1
    with torch.no_grad():
        again = newton_apply(cell, x, cfg)
    assert torch.equal(again, ref)
