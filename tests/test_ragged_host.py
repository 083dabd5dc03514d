"""Host-side rules of packed ragged batches and paged h0 (no GPU compute)."""

import pytest
import torch

from pararnn_amd.ragged import Padding, gather_h0, prepend_state_ragged, validate_cu_seqlens


@pytest.mark.parametrize("cs,time,msg", [
    ([0], 4, r"\(S\+1,\)"),
    ([1, 4], 4, r"\[0\] must be 0"),
    ([0, 3], 4, r"must equal time=4"),
    ([0, 2, 2, 4], 4, "strictly increasing"),
])
def test_validate_cu_seqlens_rejects(cs, time, msg):
    with pytest.raises(ValueError, match=msg):
        validate_cu_seqlens(torch.tensor(cs), time)


def test_padding_round_trip_and_zero_fill():
    cs = torch.tensor([0, 3, 4, 9])
    pad = Padding(cs, torch.device("cpu"))
    packed = torch.arange(1, 10, dtype=torch.float32).reshape(1, 9, 1).expand(1, 9, 2)
    p = pad.pad(packed)
    assert p.shape == (3, 5, 2)
    assert p[0, :3, 0].tolist() == [1, 2, 3] and p[0, 3:].abs().sum() == 0
    assert p[1, 0, 0] == 4 and p[1, 1:].abs().sum() == 0
    assert p[2, :, 0].tolist() == [5, 6, 7, 8, 9]
    assert torch.equal(pad.unpad(p), packed)


def test_prepend_state_ragged_heads():
    cs = torch.tensor([0, 2, 5])
    st = torch.arange(5, dtype=torch.float32).reshape(1, 5, 1)
    h0 = torch.tensor([[10.0], [20.0]])
    out = prepend_state_ragged(st, h0, cs)
    assert out[0, :, 0].tolist() == [10, 0, 20, 2, 3]
    out = prepend_state_ragged(st, None, cs)
    assert out[0, :, 0].tolist() == [0, 0, 0, 2, 3]
    with pytest.raises(ValueError, match="n_seq"):
        prepend_state_ragged(st, h0[:1], cs)


def test_gather_h0_rules():
    pool = torch.randn(4, 2, 3)
    bt = torch.tensor([3, 0])
    assert torch.equal(gather_h0(pool, bt, 2, (2, 3)), pool[bt])
    assert gather_h0(pool, None, 2, (2, 3)) is pool
    with pytest.raises(ValueError, match="outside pool"):
        gather_h0(pool, torch.tensor([0, 4]), 2, (2, 3))
    with pytest.raises(ValueError, match="B=1"):
        gather_h0(pool, torch.tensor([0]), 2, (2, 3))
    with pytest.raises(ValueError, match="tail"):
        gather_h0(pool, bt, 2, (3, 2))
    with pytest.raises(ValueError, match="needs h0"):
        gather_h0(None, bt, 2, (2, 3))


def test_newton_apply_ragged_rejects_batched_x():
    from pararnn_amd import NewtonConfig, ParaSLSTM, newton_apply

    cell = ParaSLSTM(4, 8)
    x = torch.randn(2, 6, 4)
    with pytest.raises(ValueError, match="batch=1"):
        newton_apply(cell, x, NewtonConfig(), cu_seqlens=torch.tensor([0, 6]))
    with pytest.raises(ValueError, match="chunk_len"):
        newton_apply(cell, x[:1], NewtonConfig(chunk_len=2), cu_seqlens=torch.tensor([0, 6]))
