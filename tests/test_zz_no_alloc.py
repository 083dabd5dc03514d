"""The allocation-free Newton entry point (prnn_slstm_newton_noalloc) called
through the C ABI: two calls in a row, the second on a smaller input, each
bit-equal to prnn_slstm_newton with a caller workspace on the same inputs
(both in the library's deterministic look-back mode, where a solve's result
does not depend on tile scheduling); a shape beyond the scratch maximum is
rejected with a value error before anything runs."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _inputs(B, T, d, dtype, seed):
    from pararnn_amd import ParaSLSTM, slstm_init_fused

    g = torch.Generator(device=DEV).manual_seed(seed)
    torch.manual_seed(seed)
    cell = ParaSLSTM(d, d).to(DEV, dtype)
    x = torch.randn(B, T, d, generator=g, device=DEV).to(dtype)
    h0 = torch.randn(B, 4, d, generator=g, device=DEV) * 0.5
    h0[:, 1] = h0[:, 1].abs() + 0.5
    h0 = h0.to(dtype)
    with torch.no_grad():
        wx = cell.W_x(x).contiguous()
        r = cell.clipped_r().contiguous()
        guess = slstm_init_fused(wx, r, h0, picard_iters=3, eps=cell.eps).contiguous()
    return wx, r, h0, guess, cell.eps


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _solve_pair(lib, B, T, d, K, dtype, seed):
    from pararnn_amd import _lib

    code = _lib.PRNN_BF16 if dtype == torch.bfloat16 else _lib.PRNN_F32
    wx, r, h0, guess, eps = _inputs(B, T, d, dtype, seed)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    need = lib.prnn_slstm_newton_workspace_size(B, T, d, K, code)
    assert 0 < need <= lib.prnn_slstm_newton_noalloc_max_bytes()
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    want = torch.empty_like(guess)
    got = torch.full_like(guess, float("nan"))
    print(f"case noalloc B={B} T={T} d={d} K={K} {dtype} (scratch {need} bytes)", flush=True)
    # after the torch-side ops above, which set the library's mode from
    # torch's deterministic flag
    lib.prnn_set_deterministic(1)
    _lib.check(lib.prnn_slstm_newton(_ptr(wx), _ptr(r), _ptr(h0), _ptr(guess), _ptr(want), B, T,
                                     d, K, 1.0, eps, code, _ptr(ws), need, stream),
               "prnn_slstm_newton")
    _lib.check(lib.prnn_slstm_newton_noalloc(_ptr(wx), _ptr(r), _ptr(h0), _ptr(guess), _ptr(got),
                                             B, T, d, K, 1.0, eps, code, stream),
               "prnn_slstm_newton_noalloc")
    torch.cuda.synchronize()
    return got, want


def test_noalloc_matches_workspace_entry_point_twice():
    from pararnn_amd import _lib

    lib = _lib.load()
    prev = lib.prnn_deterministic()
    try:
        got, want = _solve_pair(lib, 2, 3000, 256, 2, torch.bfloat16, 11)
        print(f"  max|noalloc - workspace| {(got.float() - want.float()).abs().max().item():.3e}",
              flush=True)
        assert torch.equal(got, want)
        # smaller, different dtype and K: the array still holds the first
        # call's look-back words, which the call must clear before use
        got, want = _solve_pair(lib, 1, 700, 70, 3, torch.float32, 12)
        print(f"  max|noalloc - workspace| {(got - want).abs().max().item():.3e}", flush=True)
        assert torch.equal(got, want)
    finally:
        lib.prnn_set_deterministic(prev)


def test_noalloc_rejects_shapes_beyond_the_scratch_maximum():
    from pararnn_amd import _lib

    lib = _lib.load()
    B, T, d, K = 1, 131072, 1024, 2
    need = lib.prnn_slstm_newton_workspace_size(B, T, d, K, _lib.PRNN_BF16)
    assert need > lib.prnn_slstm_newton_noalloc_max_bytes()
    dummy = torch.zeros(16, device=DEV)
    p = _ptr(dummy)
    rc = lib.prnn_slstm_newton_noalloc(p, p, None, p, p, B, T, d, K, 1.0, 1e-6, _lib.PRNN_BF16,
                                       None)
    assert rc == _lib.PRNN_ERR_VALUE
    assert b"scratch" in lib.prnn_last_error()
