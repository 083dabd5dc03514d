"""The torch.library ops (names and schemas of the reference's
kernels/custom_ops.py:311-540) and their fake kernels: under FakeTensorMode
each op returns the documented shapes, dtypes and device without running
anything, which is what torch.compile / Dynamo trace through
(custom_ops.py:48-51, 519-540).  CPU only: fake tensors need no GPU."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import pararnn_amd.ops  # noqa: F401  -- registers torch.ops.pararnn.*


def test_ops_registered_with_reference_names():
    for name in ("newton_slstm_fused", "newton_gru_head_fused", "slstm_init_fused",
                 "slstm_backward_fused", "gru_head_backward_fused"):
        assert hasattr(torch.ops.pararnn, name), name
    schema = str(torch.ops.pararnn.newton_slstm_fused.default._schema)
    for arg in ("Tensor wx", "Tensor r", "Tensor? h0=None", "Tensor? states=None",
                "Tensor? block_table=None", "SymInt max_iters", "float omega", "float eps",
                "bool log_coords=False", "str scan_tile=\"assoc\"", "bool time_loop=False",
                "SymInt window_len=0"):
        assert arg in schema, (arg, schema)
    schema = str(torch.ops.pararnn.newton_gru_head_fused.default._schema)
    for arg in ("Tensor wx", "Tensor a_z", "Tensor a_r", "Tensor a_n", "Tensor? h0=None",
                "Tensor? cu_seqlens=None", "SymInt max_iters", "float omega"):
        assert arg in schema, (arg, schema)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_slstm_fake_kernels(dtype):
    B, T, d = 2, 100, 64
    with FakeTensorMode():
        wx = torch.empty(B, T, 4 * d, device="cuda", dtype=dtype)
        r = torch.empty(4, d, device="cuda", dtype=dtype)
        h0 = torch.empty(B, 4, d, device="cuda", dtype=dtype)
        guess = torch.ops.pararnn.slstm_init_fused(wx, r, h0, picard_iters=5, eps=1e-6)
        assert guess.shape == (B, T, 4, d) and guess.dtype == dtype and guess.device.type == "cuda"
        out = torch.ops.pararnn.newton_slstm_fused(wx, r, h0, guess, None, max_iters=2,
                                                   omega=1.0, eps=1e-6)
        assert out.shape == (B, T, 4, d) and out.dtype == dtype
        out0 = torch.ops.pararnn.newton_slstm_fused(wx, r, None, None, None, max_iters=2,
                                                    omega=1.0, eps=1e-6)
        assert out0.shape == (B, T, 4, d)
        g_wx, g_r, g_h0, g_b = torch.ops.pararnn.slstm_backward_fused(wx, r, h0, out, out,
                                                                      eps=1e-6)
        assert g_b.shape == (4, d) and g_b.dtype == torch.float32
        assert g_wx.shape == wx.shape and g_wx.dtype == dtype
        assert g_r.shape == (4, d) and g_r.dtype == torch.float32
        assert g_h0.shape == (B, 4, d) and g_h0.dtype == torch.float32


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gru_head_fake_kernels(dtype):
    B, T, H = 2, 70, 3
    d = 64 * H
    with FakeTensorMode():
        wx = torch.empty(B, T, 3 * d, device="cuda", dtype=dtype)
        a = [torch.empty(H, 64, 64, device="cuda", dtype=dtype) for _ in range(3)]
        h0 = torch.empty(B, d, device="cuda", dtype=dtype)
        out = torch.ops.pararnn.newton_gru_head_fused(wx, *a, h0, None, max_iters=3, omega=1.0)
        assert out.shape == (B, T, d) and out.dtype == dtype and out.device.type == "cuda"
        g_wx, g_a, g_h0 = torch.ops.pararnn.gru_head_backward_fused(wx, *a, h0, out, out)
        assert g_wx.shape == wx.shape and g_wx.dtype == dtype
        assert g_a.shape == (3, H, 64, 64) and g_a.dtype == torch.float32
        assert g_h0.shape == (B, d) and g_h0.dtype == torch.float32


def test_precision_region_disables_autocast():
    """The solve runs outside an outer autocast (newton/__init__.py:193-209)."""
    from pararnn_amd.newton import _newton_precision_region

    with torch.autocast(device_type="cpu", dtype=torch.bfloat16):
        assert torch.is_autocast_enabled("cpu")
        with _newton_precision_region(torch.device("cpu")):
            assert not torch.is_autocast_enabled("cpu")
            y = torch.nn.functional.linear(torch.randn(3, 4), torch.randn(5, 4))
            assert y.dtype == torch.float32
        assert torch.is_autocast_enabled("cpu")


def test_tagged_workspace_cache_is_bounded(monkeypatch):
    """One zero-filled buffer per (device, stream), at most a few kept, tag
    bases 64 apart and growing; no GPU needed (buffers made on the CPU)."""
    from pararnn_amd import ops

    made = []
    real_zeros = torch.zeros

    def fake_zeros(n, dtype, device):
        made.append(n)
        return real_zeros(n, dtype=dtype)

    class _S:
        def __init__(self, h):
            self.cuda_stream = h

    monkeypatch.setattr(ops.torch, "zeros", fake_zeros)
    monkeypatch.setattr(ops.torch.cuda, "is_current_stream_capturing", lambda: False)
    ops.release_workspaces()
    dev = torch.device("cuda", 0)
    bases = []
    for h in range(10):
        monkeypatch.setattr(ops.torch.cuda, "current_stream", lambda d, h=h: _S(1000 + h))
        ws, base = ops._slstm_workspace(1024, dev)
        ws2, base2 = ops._slstm_workspace(512, dev)  # same stream: same buffer, next base
        assert ws2 is ws and base2 == base + ops._TAG_SPAN
        bases.append(base)
    assert len(ops._tagged) == ops._TAGGED_MAX
    assert all(b == 1 for b in bases) and len(made) == 10
    ops.release_workspaces()
    assert not ops._tagged
