"""``ParaRNN`` host logic on the CPU: reference checkpoints load by name, the
eval() (sequential) path matches the reference's output, and the reference's
validation rules hold."""

import pytest
import torch
from conftest import load_golden

from pararnn_amd import NewtonConfig, ParaGRU, ParaRNN, ParaSLSTM


def _model(name):
    t, m = load_golden(name)
    if m["cell"] == "slstm":
        cell = ParaSLSTM(m["d_in"], m["d"])
    else:
        cell = ParaGRU(m["d_in"], m["d"], mix="head", n_heads=m["n_heads"])
    cfg = NewtonConfig(max_iters=m["K"], picard_iters=m["P"], residual_atol=None,
                       residual_fail=None, picard_adapt=False)
    model = ParaRNN(cell, num_layers=m["layers"], config=cfg, return_hidden=True)
    sd = {k[3:]: v for k, v in t.items() if k.startswith("sd.")}
    model.load_state_dict(sd, strict=True)  # same parameter names and shapes
    return model, t, m


@pytest.mark.parametrize("name", ["para_rnn_slstm_fp32", "para_rnn_gru_head_fp32"])
def test_eval_path_matches_reference(name):
    model, t, _ = _model(name)
    model.eval()
    with torch.no_grad():
        y, last = model(t["x"])
    assert torch.allclose(y, t["y_seq"], rtol=0, atol=2e-6)
    assert torch.allclose(last, t["last_seq"], rtol=0, atol=2e-6)


def test_validation_rules():
    with pytest.raises(ValueError, match="solver"):
        ParaRNN(ParaSLSTM(4, 8), solver="fast")
    with pytest.raises(ValueError, match="dropout"):
        ParaRNN(ParaSLSTM(4, 8), dropout=1.5)
    with pytest.raises(TypeError, match="ParaLSTM"):
        ParaRNN(ParaSLSTM(4, 8), hidden_layout="pytorch")
    with pytest.raises(ValueError, match="num_layers"):
        ParaRNN([ParaSLSTM(4, 8), ParaSLSTM(8, 8)], num_layers=3)
    with pytest.warns(UserWarning, match="dropout"):
        ParaRNN(ParaSLSTM(4, 8), dropout=0.2)
    m = ParaRNN(ParaSLSTM(4, 8), num_layers=2).eval()
    with pytest.raises(ValueError, match="expected input features 4"):
        m(torch.randn(1, 3, 5))
    with pytest.raises(TypeError, match="length 2"):
        m(torch.randn(1, 3, 4), h0=torch.zeros(1, 4, 8))
    with pytest.raises(ValueError, match=r"h0 for layer 1 expected shape \(1, 4, 8\)"):
        m(torch.randn(1, 3, 4), h0=[None, torch.zeros(1, 8)])
    # stacking keeps the cell's knobs, deeper layers take hidden -> hidden
    g = ParaRNN(ParaGRU(4, 128, mix="head", n_heads=2), num_layers=3)
    assert [c.input_size for c in g.layers] == [4, 128, 128]
    assert all(c.mix == "head" and c.n_heads == 2 for c in g.layers)


def test_layout_and_packed_eval():
    torch.manual_seed(0)
    m = ParaRNN(ParaSLSTM(4, 8), num_layers=2, batch_first=False).eval()
    x = torch.randn(7, 3, 4)
    with torch.no_grad():
        y = m(x)
        m.batch_first = True
        y2 = m(x.transpose(0, 1))
    assert y.shape == (7, 3, 8) and torch.allclose(y.transpose(0, 1), y2)
    # packed sequences = the per-sequence runs laid end to end
    xs = torch.randn(1, 9, 4)
    cs = torch.tensor([0, 4, 9])
    with torch.no_grad():
        yp = m(xs, cu_seqlens=cs)
        ya = m(xs[:, :4])
        yb = m(xs[:, 4:])
    assert torch.allclose(yp, torch.cat([ya, yb], 1), atol=1e-6)
