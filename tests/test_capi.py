"""The C-ABI library loads and exports every entry point include/pararnn_amd.h
declares, with the argument counts the ctypes binding uses.  No GPU calls."""

import ctypes
import os
import re

import pytest
from conftest import REPO


def _declared():
    text = open(os.path.join(REPO, "include", "pararnn_amd.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"PRNN_API\s+[\w\s\*]+?\b(prnn_\w+)\s*\(([^)]*)\)", text):
        args = [a for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        out[m.group(1)] = len(args)
    return out


def test_header_declares_entry_points():
    decl = _declared()
    for name in ("prnn_slstm_init", "prnn_slstm_newton", "prnn_gru_head_newton",
                 "prnn_slstm_backward", "prnn_gru_head_backward", "prnn_slstm_decode",
                 "prnn_gru_decode", "prnn_last_error", "prnn_abi_version",
                 "prnn_set_deterministic", "prnn_deterministic", "prnn_set_kernel_timing",
                 "prnn_last_kernel_ms", "prnn_slstm_init_ex", "prnn_slstm_newton_ex",
                 "prnn_slstm_backward_ex"):
        assert name in decl


def test_library_exports_every_declared_symbol():
    from pararnn_amd import _lib

    if not os.path.exists(_lib.lib_path()):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.lib_path())
    decl = _declared()
    for name, nargs in decl.items():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, name
        assert len(_lib.SIGNATURES[name][1]) == nargs, name


def test_host_only_calls():
    from pararnn_amd import _lib

    if not os.path.exists(_lib.lib_path()):
        pytest.skip("library not built")
    lib = _lib.load()
    assert lib.prnn_abi_version() == _lib.ABI_VERSION
    lib.prnn_set_deterministic(1)
    assert lib.prnn_deterministic() == 1
    lib.prnn_set_deterministic(0)
    assert lib.prnn_deterministic() == 0
    assert lib.prnn_last_kernel_ms() == -1.0  # nothing timed yet
    n = lib.prnn_slstm_newton_workspace_size(1, 131072, 1024, 2, _lib.PRNN_BF16)
    # K >= 2 runs in one launch: look-back words per iteration, no fp32
    # trajectory in memory; more iterations need more words.
    assert 0 < n < 131072 * 4 * 1024 * 4
    assert lib.prnn_slstm_newton_workspace_size(1, 131072, 1024, 3, _lib.PRNN_BF16) > n
    assert lib.prnn_slstm_newton_workspace_size(0, 1, 1, 2, 0) == 0
    assert lib.prnn_slstm_init_workspace_size(1, 10, 10, -1, 0) == 0
    # invalid arguments fail before any device work
    rc = lib.prnn_slstm_newton(None, None, None, None, None, 1, 1, 1, 1, 1.0, 1e-6, 0,
                               None, 0, None)
    assert rc == _lib.PRNN_ERR_VALUE
    assert b"non-null" in lib.prnn_last_error()
    rc = lib.prnn_slstm_init(None, None, None, None, 1, 1, 1, 0, 1e-6, 7, None, 0, None)
    assert rc == _lib.PRNN_ERR_TYPE
    with pytest.raises(TypeError):
        _lib.check(rc, "x")
    assert lib.prnn_slstm_backward_workspace_size(4, 32768, 768, _lib.PRNN_BF16) > 0
    rc = lib.prnn_slstm_backward(None, None, None, None, None, None, None, None, 1, 1, 1, 1e-6,
                                 0, None, 0, None)
    assert rc == _lib.PRNN_ERR_VALUE
    assert lib.prnn_gru_head_backward_workspace_size(4, 32768, 8, 64, _lib.PRNN_F32) > 0
    assert lib.prnn_gru_head_backward_workspace_size(4, 32768, 8, 32, _lib.PRNN_F32) == 0
    rc = lib.prnn_gru_head_backward(None, None, None, None, None, None, None, None, None, None,
                                    1, 1, 1, 64, 0, None, 0, None)
    assert rc == _lib.PRNN_ERR_VALUE
    rc = lib.prnn_slstm_newton_ex(None, None, None, None, None, 1, 1, 1, 1, 1.0, 1e-6, 0,
                                  None, 0, -1, None)
    assert rc == _lib.PRNN_ERR_VALUE and b"tag_base" in lib.prnn_last_error()
    rc = lib.prnn_slstm_init_ex(None, None, None, None, 1, 1, 1, 0, 1e-6, 0, None, 0,
                                (1 << 30) + 1, None)
    assert rc == _lib.PRNN_ERR_VALUE and b"tag_base" in lib.prnn_last_error()
    rc = lib.prnn_slstm_backward_ex(None, None, None, None, None, None, None, None, None, 1, 1, 1,
                                    1e-6, 0, None, 0, 5, None)
    assert rc == _lib.PRNN_ERR_VALUE and b"non-null" in lib.prnn_last_error()


def test_packed_entry_points_reject_bad_sequence_counts():
    """n_seq outside [1, T] cannot describe strictly rising offsets of a
    T-step stream: every packed entry point rejects it before any device
    work (cu_seqlens is never read, so a dummy address is enough)."""
    from pararnn_amd import _lib

    if not os.path.exists(_lib.lib_path()):
        pytest.skip("library not built")
    lib = _lib.load()
    cu = 64  # never dereferenced: the size check fails first
    for n_seq in (0, 11):
        rc = lib.prnn_slstm_init_packed(None, None, None, None, 10, 4, 1, 1e-6, 0, cu, n_seq,
                                        None, None, 0, 0, None)
        assert rc == _lib.PRNN_ERR_VALUE and b"n_seq" in lib.prnn_last_error()
        rc = lib.prnn_slstm_newton_packed(None, None, None, None, None, 10, 4, 2, 1.0, 1e-6, 0,
                                          cu, n_seq, None, None, 0, 0, None)
        assert rc == _lib.PRNN_ERR_VALUE and b"n_seq" in lib.prnn_last_error()
        rc = lib.prnn_slstm_newton_step_packed(None, None, None, None, 0, None, 10, 4, 1.0, 1e-6,
                                               0, cu, n_seq, None, None, 0, 0, None)
        assert rc == _lib.PRNN_ERR_VALUE and b"n_seq" in lib.prnn_last_error()
        rc = lib.prnn_slstm_backward_packed(None, None, None, None, None, None, None, None, None,
                                            10, 4, 1e-6, 0, cu, n_seq, None, 0, 0, None)
        assert rc == _lib.PRNN_ERR_VALUE and b"n_seq" in lib.prnn_last_error()
        rc = lib.prnn_gru_head_newton_packed(None, None, None, None, None, None, 10, 1, 64, 2,
                                             1.0, 0, cu, n_seq, None, None, 0, None)
        assert rc == _lib.PRNN_ERR_VALUE and b"n_seq" in lib.prnn_last_error()


def test_one_iteration_workspace_covers_the_short_tiles():
    """A max_iters = 1 workspace also serves the single-iteration launches (the
    residual-gated step and the eager iteration), whose tiles can be shorter
    than the fused launch's: its look-back words (4 inclusive + 20 aggregate
    8-byte words per channel and tile) must cover the shortest 16-bit tiles of
    those launches, 32 steps on packed streams (8 x 4 waves) and 48 steps on
    rectangular batches (12 x 4)."""
    from pararnn_amd import _lib

    if not os.path.exists(_lib.lib_path()):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = _lib.load()
    bf16 = 1

    def words(T, d, steps):
        return 24 * 8 * 64 * (-(-T // steps) * -(-d // 64))

    for T, d in ((131072, 1024), (4099, 192), (64, 64)):
        assert lib.prnn_slstm_newton_packed_workspace_size(T, d, 1, bf16) >= words(T, d, 32)
        assert lib.prnn_slstm_newton_workspace_size(1, T, d, 1, bf16) >= words(T, d, 48)
        assert lib.prnn_slstm_newton_workspace_size(4, T, d, 1, bf16) >= 4 * words(T, d, 48)
