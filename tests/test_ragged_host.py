"""Host-side rules of packed ragged batches and paged h0 (no GPU compute)."""

import pytest
import torch

from pararnn_amd.ragged import (
    Padding,
    RaggedPlan,
    gather_h0,
    length_groups,
    prepend_state_ragged,
    validate_cu_seqlens,
)


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


def test_length_groups_bound_padding():
    g = torch.Generator().manual_seed(0)
    lengths = [int(v) for v in torch.randint(1, 5000, (200,), generator=g)] + [100000, 3]
    groups = length_groups(lengths)
    assert sorted(i for grp in groups for i in grp) == list(range(len(lengths)))
    for grp in groups:
        top = max(lengths[i] for i in grp)
        assert all(top <= max(2 * lengths[i], lengths[i] + 256) for i in grp)
    # one rectangle would cost 202 * 100000 steps; the groups stay near 2 N
    padded = sum(len(grp) * max(lengths[i] for i in grp) for grp in groups)
    assert padded <= 2 * sum(lengths) + 256 * len(lengths)
    assert len(groups) <= 12
    # near-uniform lengths stay one rectangle
    assert len(length_groups([4096, 4000, 3000, 2100])) == 1


def _solve_marker(padded, h0):
    """A stand-in solve: every step of row s gets its input plus h0[s]; the
    padded rectangle must be (S_g, T_g, ...) with the group's own h0 rows."""
    assert h0 is None or h0.shape[0] == padded.shape[0]
    return padded if h0 is None else padded + h0[:, None]


@pytest.mark.parametrize("lengths", [[3, 1, 5], [700, 5, 2, 1300, 40, 9000, 3]])
def test_ragged_plan_packed_order(lengths, monkeypatch):
    cs = torch.tensor([0] + lengths).cumsum(0)
    n = int(cs[-1])
    packed = torch.randn(1, n, 3, requires_grad=True)
    h0 = torch.randn(len(lengths), 3)
    want = packed.detach() + h0.repeat_interleave(torch.tensor(lengths), 0)[None]
    plan = RaggedPlan(cs, torch.device("cpu"))
    assert plan.n_groups == (1 if max(lengths) < 600 else 3)
    assert plan.padded_steps <= 2 * n + 256 * len(lengths)
    out = plan.run(packed, h0, _solve_marker)
    assert torch.equal(out, want)
    out.mul(torch.arange(n, dtype=torch.float32)[None, :, None]).sum().backward()
    assert torch.equal(packed.grad[0, :, 0], torch.arange(n, dtype=torch.float32))
    monkeypatch.setenv("PARARNN_AMD_RAGGED_GROUPS", "0")
    single = RaggedPlan(cs, torch.device("cpu"))
    assert single.n_groups == 1 and single.padded_steps == len(lengths) * max(lengths)
    assert torch.equal(single.run(packed.detach(), h0, _solve_marker), want)


def test_validated_offsets_are_checked_again_after_a_write():
    """The solve checks one stream once; an in-place write to the offsets (or
    another length) makes the next call check them again."""
    cs = torch.tensor([0, 3, 7], dtype=torch.int32)
    out = validate_cu_seqlens(cs, 7)
    assert out.dtype == torch.long and out.tolist() == [0, 3, 7]
    assert validate_cu_seqlens(out, 7) is out
    cs[1] = 9
    with pytest.raises(ValueError, match="strictly increasing"):
        validate_cu_seqlens(cs, 7)
    cs[1] = 3
    validate_cu_seqlens(cs, 7)
    with pytest.raises(ValueError, match="must equal time"):
        validate_cu_seqlens(cs, 8)
