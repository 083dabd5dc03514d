"""Host logic of the determinism check (pararnn/determinism.py:41-113 of the
reference): the byte-level bit-match and the one-shot re-run warning."""

import logging

import torch

from pararnn_amd import determinism


def test_bitmatch():
    a = torch.tensor([1.0, float("nan"), -0.0])
    assert determinism.param_grads_bitmatch((a, None), (a.clone(), None))
    assert not determinism.param_grads_bitmatch((a,), (torch.tensor([1.0, float("nan"), 0.0]),))
    b = a.clone()
    b[0] = torch.nextafter(torch.tensor(1.0), torch.tensor(2.0))
    assert not determinism.param_grads_bitmatch((a,), (b,))
    assert not determinism.param_grads_bitmatch((a, None), (a, a))
    assert not determinism.param_grads_bitmatch((a,), (a, a))
    assert not determinism.param_grads_bitmatch((a,), (a.to(torch.float64),))


def test_one_shot_warning(caplog):
    prev = torch.are_deterministic_algorithms_enabled()
    calls = []

    def rerun():
        calls.append(1)
        return (torch.ones(3) * (1 + len(calls)),)

    try:
        determinism.reset_checks()
        torch.use_deterministic_algorithms(False)
        determinism.maybe_check_fused_vjp_once((torch.ones(3),), rerun, cell_name="C", shape=(1,))
        assert calls == []  # flag off: nothing re-run
        torch.use_deterministic_algorithms(True, warn_only=True)
        with caplog.at_level(logging.WARNING, logger="pararnn_amd"):
            determinism.maybe_check_fused_vjp_once((torch.ones(3),), rerun, cell_name="C",
                                                   shape=(1,))
            determinism.maybe_check_fused_vjp_once((torch.ones(3),), rerun, cell_name="C",
                                                   shape=(1,))
        assert calls == [1]  # only the first VJP is re-run
        msgs = [r.getMessage() for r in caplog.records if "differed" in r.getMessage()]
        assert len(msgs) == 1 and "cell=C" in msgs[0]
        determinism.reset_checks()
        caplog.clear()
        with caplog.at_level(logging.WARNING, logger="pararnn_amd"):
            determinism.maybe_check_fused_vjp_once(
                (torch.ones(3),), lambda: (torch.ones(3),), cell_name="C", shape=(1,))
        assert not caplog.records
    finally:
        torch.use_deterministic_algorithms(prev)
        determinism.reset_checks()
