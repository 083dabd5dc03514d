"""GPU parity of ``ParaRNN`` (stacked cells) against the reference's outputs:
train() runs the fused Newton solve per layer, eval() the sequential unroll."""

import pytest
import torch
from conftest import load_golden

from pararnn_amd import NewtonConfig, ParaGRU, ParaRNN, ParaSLSTM, verify_agreement

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.mark.parametrize("name", ["para_rnn_slstm_fp32", "para_rnn_gru_head_fp32"])
def test_train_and_eval_match_reference(name):
    print(f"case ParaRNN {name}", flush=True)
    t, m = load_golden(name)
    if m["cell"] == "slstm":
        cell = ParaSLSTM(m["d_in"], m["d"])
    else:
        cell = ParaGRU(m["d_in"], m["d"], mix="head", n_heads=m["n_heads"])
    cfg = NewtonConfig(max_iters=m["K"], picard_iters=m["P"], residual_atol=None,
                       residual_fail=None, picard_adapt=False)
    model = ParaRNN(cell, num_layers=m["layers"], config=cfg, return_hidden=True)
    model.load_state_dict({k[3:]: v for k, v in t.items() if k.startswith("sd.")})
    model = model.to(DEV)
    x = t["x"].to(DEV)
    with torch.no_grad():
        model.train()
        y, last = model(x)
        model.eval()
        ys, lasts = model(x)
    e_new = (y.cpu() - t["y_newton"]).abs().max().item()
    e_seq = (ys.cpu() - t["y_seq"]).abs().max().item()
    print(f"  newton max|gpu-ref| {e_new:.2e}, sequential {e_seq:.2e}", flush=True)
    assert e_new <= 1e-5 and e_seq <= 1e-5
    assert (last.cpu() - t["last_newton"]).abs().max().item() <= 3e-5
    assert len(model.last_stats) == 0 or all(s.iters == m["K"] for s in model.last_stats)
    rep = verify_agreement(model, x)
    print(f"  verify_agreement(ParaRNN) max_abs {rep.max_abs:.2e} path {rep.path}", flush=True)
    assert rep.path == "para_rnn" and rep.ok


def test_train_backward_through_stack():
    print("case ParaRNN 2-layer sLSTM backward vs float64 sequential autograd", flush=True)
    torch.manual_seed(3)
    model = ParaRNN(ParaSLSTM(8, 32), num_layers=2,
                    config=NewtonConfig(max_iters=6, picard_iters=3, residual_atol=None,
                                        residual_fail=None, picard_adapt=False)).to(DEV)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 90, 8, generator=g)
    up = torch.randn(2, 90, 32, generator=g)
    xd = x.to(DEV).requires_grad_(True)
    model.train()
    (model(xd) * up.to(DEV)).sum().backward()
    ref = ParaRNN([c.__class__(c.input_size, c.hidden_size) for c in model.layers],
                  solver="sequential").double()
    ref.load_state_dict({k: v.detach().cpu().double() for k, v in model.state_dict().items()})
    x64 = x.double().requires_grad_(True)
    (ref(x64) * up.double()).sum().backward()
    e = (xd.grad.cpu().double() - x64.grad).abs().max().item() / x64.grad.abs().max().item()
    print(f"  x grad rel {e:.2e}", flush=True)
    assert e <= 1e-4
    for (n, p), (_, q) in zip(model.named_parameters(), ref.named_parameters()):
        e = (p.grad.cpu().double() - q.grad).abs().max().item() / q.grad.abs().max().item()
        print(f"  {n}: rel {e:.2e}", flush=True)
        assert e <= 1e-4, n
