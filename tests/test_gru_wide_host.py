"""Host-side pieces of the wide-head GRU tier (64 < d_head <= 128) that run
without a GPU: the previous-state layout with and without packed sequences,
and the argument checks of the one-launch entry point."""

import torch


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


def test_gates_entry_refuses_bad_arguments():
    """prnn_gru_wide_gates checks sizes, dtype and pointers before launching."""
    import ctypes
    import os

    import pytest
    from pararnn_amd import _lib

    if not os.path.exists(_lib.lib_path()):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = _lib.load()
    p = ctypes.c_void_p(4096)

    def call(rows=10, H=2, dh=96, dtype=0, z=p):
        return lib.prnn_gru_wide_gates(p, p, p, p, p, z, p, p, rows, H, dh, dtype, None)

    for rc in (call(rows=0), call(H=0), call(dh=0), call(dh=129), call(dtype=7), call(z=None)):
        assert rc != 0
