"""The fused solves under HIP graph capture: each captured graph is replayed
several times, with eager work and synchronisations in between, and every
replay is checked against the eager result.  The look-back words are cleared
by a fill kernel (no memset node), so replays start from clean state."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up outside capture (library load, workspace sizes)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


def test_slstm_fused_solve_graph_replay():
    from pararnn_amd import ParaSLSTM, fused_newton

    print("case graph: sLSTM bf16 warm start + fused K=2 Newton, 4 replays", flush=True)
    torch.manual_seed(0)
    cell = ParaSLSTM(64, 256).to(DEV, torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(1)
    x = (torch.randn(2, 4096, 64, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    with torch.no_grad():
        wx = cell.W_x(x)
        run = lambda: fused_newton(cell, wx, max_iters=2, omega=1.0, h0=None, picard_iters=3)
        eager = run().float()
        graph, out = _capture(run)
        for i in range(4):
            out.zero_()
            _ = run()  # eager work between replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            rel = ((out.float() - eager).abs() / (eager.abs() + 1e-3)).max().item()
            print(f"  replay {i}: max rel diff vs eager {rel:.2e}", flush=True)
            # look-back composition order may differ in the last bits (bf16 ulp)
            assert rel <= 2 ** -6


def test_gru_head_solve_graph_replay_bit_equal():
    from pararnn_amd import ParaGRU, fused_newton

    print("case graph: head GRU fp32 K=3, 4 replays, bit-equal", flush=True)
    torch.manual_seed(2)
    cell = ParaGRU(32, 256, mix="head", n_heads=4).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn(2, 2000, 32, generator=g, device=DEV)
    h0 = torch.randn(2, 256, generator=g, device=DEV) * 0.5
    with torch.no_grad():
        wx = cell.W_x(x)
        run = lambda: fused_newton(cell, wx, max_iters=3, omega=1.0, h0=h0)
        eager = run().clone()
        graph, out = _capture(run)
        for i in range(4):
            out.zero_()
            _ = run()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), i


def test_wide_head_one_launch_graph_replay_bit_equal():
    """d_head = 128, K = 3: the one-launch wide solve (ticket counters and the
    tagged iterates cleared by a fill kernel inside the graph) replays bit
    for bit."""
    from pararnn_amd import ParaGRU, fused_newton

    print("case graph: wide heads fp32 K=3 one launch, 4 replays, bit-equal", flush=True)
    torch.manual_seed(4)
    cell = ParaGRU(32, 256, mix="head", n_heads=2).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(2, 1500, 32, generator=g, device=DEV)
    h0 = torch.randn(2, 256, generator=g, device=DEV) * 0.5
    with torch.no_grad():
        wx = cell.W_x(x)
        run = lambda: fused_newton(cell, wx, max_iters=3, omega=1.0, h0=h0)
        eager = run().clone()
        graph, out = _capture(run)
        for i in range(4):
            out.zero_()
            _ = run()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), i
