"""Host-side pieces of the wide-head GRU tier (64 < d_head <= 128) that run
without a GPU: the gates the host computes before each HIP walk, against the
oracle's head cell (reference cells/para_gru.py:414-467), and the
previous-state layout with and without packed sequences."""

import torch

import oracle as O
from oracle.gru_head import _acts


def test_wide_gates_match_the_oracle_cell():
    from pararnn_amd.ops import _wide_gates, _wide_prev

    g = torch.Generator().manual_seed(0)
    H, dh, B, T = 2, 96, 2, 17
    d = H * dh
    p = O.GRUHeadParams(torch.randn(3 * d, 5, generator=g), torch.randn(3 * d, generator=g),
                        *(torch.randn(H, dh, dh, generator=g) * 0.1 for _ in range(3)))
    wx = torch.randn(B, T, 3 * d, generator=g)
    states = torch.randn(B, T, d, generator=g)
    h0 = torch.randn(B, d, generator=g)
    hp = _wide_prev(states, h0, None)
    assert torch.equal(hp[:, 0], h0) and torch.equal(hp[:, 1:], states[:, :-1])
    z, r, n = _wide_gates(wx, hp, p.mats())
    a = _acts(p, hp, wx)
    for got, want in ((z, a["z"]), (r, a["r"]), (n, a["n"])):
        assert (got - want.reshape(B, T, d)).abs().max().item() <= 1e-6
    new = torch.lerp(hp, n, z)
    assert (new - a["new"]).abs().max().item() <= 1e-6


def test_wide_prev_of_a_packed_stream():
    from pararnn_amd.ops import _wide_prev

    states = torch.arange(10.0).view(1, 10, 1).expand(1, 10, 3).contiguous()
    cs = torch.tensor([0, 4, 5, 10])
    h0 = torch.tensor([[-1.0] * 3, [-2.0] * 3, [-3.0] * 3])
    hp = _wide_prev(states, h0, cs)
    assert hp[0, :, 0].tolist() == [-1, 0, 1, 2, -2, -3, 5, 6, 7, 8]
    assert _wide_prev(states, None, cs)[0, :, 0].tolist() == [0, 0, 1, 2, 0, 0, 5, 6, 7, 8]


def test_one_launch_newton_entry_refuses_bad_arguments():
    """prnn_gru_wide_newton checks its arguments before touching the device:
    the iteration range, aliasing of the guess by the output, null pointers
    and the workspace size (no compute calls: pointers are never dereferenced
    on the error paths)."""
    import ctypes
    import os

    import pytest
    from pararnn_amd import _lib

    if not os.path.exists(_lib.lib_path()):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = _lib.load()
    B, T, H, dh = 2, 50, 2, 96
    need = lib.prnn_gru_wide_newton_workspace_size(B, T, H, dh, 3)
    # counters + two tagged iterates of B*T*d 64-bit words
    assert need >= 2 * B * T * H * dh * 8
    assert lib.prnn_gru_wide_newton_workspace_size(B, T, H, dh, 0) == 0
    fake = ctypes.c_void_p(4096)
    other = ctypes.c_void_p(8192)

    def call(K=3, guess=fake, out=other, ws_bytes=need, dh_=dh):
        return lib.prnn_gru_wide_newton(fake, fake, fake, fake, None, guess, out, B, T, H, dh_,
                                        K, 1.0, 0, None, 0, fake, ws_bytes, 0, None)

    for rc in (call(K=0), call(K=65), call(out=fake), call(guess=None),
               call(ws_bytes=need - 1), call(dh_=129)):
        assert rc != 0
