"""Write golden input/output vectors from the reference's eager CPU path.

The reference ships no tests, fixtures or known-answer vectors, and the exact
rounding of its eager path (bf16 re-rounding after every torch op, the fp32
Blelloch summation order, the cumsum/cummax stabiliser of the frozen-gate
scan, and the resolved Picard depth) is not fixed by any closed form.  This
script therefore imports the reference ONCE, in the build container (never on
the GPU box), and stores small safetensors fixtures next to itself.  The
fixtures are data only: inputs, weights and the reference's outputs.

Run:  PYTHONPATH=/root/reference/src python tests/golden/make_golden.py [case ...]

Reference call sites exercised (paths relative to the reference's src/pararnn):
  solvers/newton/__init__.py:212 newton_apply   (scan_backend='eager')
  solvers/sequential.py:22       sequential_apply
  solvers/slstm_picard.py:160    slstm_picard_init
  solvers/scan.py:82,103         scan_block4 / scan_dense
  cells/para_slstm.py:241        ParaSLSTM.step_with_jacobian
  cells/para_gru.py:344          ParaGRU.step_with_jacobian
  solvers/newton/__init__.py:91  _NewtonFixedPoint (eq. 2.6 backward, eager)
  solvers/scan.py:166            reverse_scan_block4
  kernels/vjp_slstm.py:173       slstm_recurrence_vjp_eager
  kernels/gru_head_factor.py:68  gru_head_jt_mvp
  kernels/vjp_gru.py:141         gru_head_recurrence_vjp_eager
  layers/para_rnn.py:27          ParaRNN (train: Newton, eval: sequential)
"""

from __future__ import annotations

import json
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))


def _save(name: str, tensors: dict, meta: dict) -> None:
    out = {k: v.detach().contiguous().cpu() for k, v in tensors.items()}
    path = os.path.join(HERE, f"{name}.safetensors")
    save_file(out, path, metadata={"meta": json.dumps(meta)})
    size = os.path.getsize(path)
    print(f"wrote {path} ({size / 1e6:.2f} MB)")


def _cfg(K: int, P: int | None):
    from pararnn import NewtonConfig

    return NewtonConfig(
        max_iters=K,
        residual_atol=None,
        residual_fail=None,
        picard_iters=P,
        picard_adapt=False,
        scan_backend="eager",
    )


def slstm_case(name, *, d_in, d, B, T, K, P, dtype, seed, x_std=1.0, with_h0=False,
               keep_wx=True):
    from pararnn import ParaSLSTM, newton_apply, sequential_apply
    from pararnn.solvers.slstm_picard import slstm_picard_init

    torch.manual_seed(seed)
    cell = ParaSLSTM(d_in, d, mix="diag")
    cell = cell.to(dtype)
    g = torch.Generator().manual_seed(seed + 1)
    x = (torch.randn(B, T, d_in, generator=g) * x_std).to(dtype)
    h0 = None
    tensors = {}
    if with_h0:
        # A reachable state: the sequential unroll of a short random prefix.
        xp = torch.randn(B, 16, d_in, generator=g).to(dtype)
        with torch.no_grad():
            h0 = sequential_apply(cell, xp)[:, -1].clone()
        tensors["h0"] = h0
    with torch.no_grad():
        wx = cell.W_x(x)
        init = slstm_picard_init(cell, wx, h0=h0, n_picard=P)
        H = newton_apply(cell, x, _cfg(K, P), h0=h0)
        Hs = sequential_apply(cell, x, h0)
    tensors.update(
        x=x,
        W=cell.W_x.weight,
        b=cell.W_x.bias,
        R=cell.R,
        wx=wx,
        init=init,
        newton=H,
        sequential=Hs,
    )
    if not keep_wx:
        # fp32 wx is recomputed exactly from x, W, b; dropping it keeps the file small.
        tensors.pop("wx")
    meta = dict(cell="ParaSLSTM", mix="diag", d_in=d_in, d=d, B=B, T=T, K=K, P=P,
                dtype=str(dtype).replace("torch.", ""), seed=seed, x_std=x_std,
                eps=cell.eps, max_recurrent_norm=cell.max_recurrent_norm, h0=with_h0)
    _save(name, tensors, meta)


def gru_head_case(name, *, d_in, n_heads, d_head, B, T, K, dtype, seed, with_h0=False):
    from pararnn import ParaGRU, newton_apply, sequential_apply

    torch.manual_seed(seed)
    cell = ParaGRU(d_in, n_heads * d_head, mix="head", n_heads=n_heads)
    cell = cell.to(dtype)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(B, T, d_in, generator=g).to(dtype)
    h0 = None
    tensors = {}
    if with_h0:
        h0 = (0.5 * torch.randn(B, n_heads * d_head, generator=g)).to(dtype)
        tensors["h0"] = h0
    with torch.no_grad():
        wx = cell.W_x(x)
        H = newton_apply(cell, x, _cfg(K, None), h0=h0)
        Hs = sequential_apply(cell, x, h0)
    tensors.update(
        x=x, W=cell.W_x.weight, b=cell.W_x.bias, A_z=cell.A_z, A_r=cell.A_r, A_n=cell.A_n,
        wx=wx, newton=H, sequential=Hs,
    )
    meta = dict(cell="ParaGRU", mix="head", d_in=d_in, n_heads=n_heads, d_head=d_head,
                B=B, T=T, K=K, dtype=str(dtype).replace("torch.", ""), seed=seed, h0=with_h0)
    _save(name, tensors, meta)


def parts_case():
    """Single-step cell/Jacobian values and bare scans on random operands."""
    from pararnn import ParaGRU, ParaSLSTM
    from pararnn.solvers.scan import scan_block4, scan_dense
    from pararnn.solvers.slstm_picard import slstm_frozen_gate_scan_eager

    g = torch.Generator().manual_seed(1234)
    torch.manual_seed(1234)
    cell = ParaSLSTM(8, 16, mix="diag")
    state = torch.randn(3, 5, 4, 16, generator=g)
    state[..., 1, :] = state[..., 1, :].abs() + 0.1  # normaliser n > 0
    wx = torch.randn(3, 5, 64, generator=g)
    # Force exact ties of the maximum in a few places (0.5/0.5 subgradient).
    r = cell.clipped_r().detach()
    h = state[..., 3, :]
    pre_f = wx[..., 16:32] + r[1] * h
    wx[..., 0, 0, 0:4] = (pre_f[0, 0, 0:4] + state[0, 0, 2, 0:4]) - r[0, 0:4] * h[0, 0, 0:4]
    with torch.no_grad():
        new, jac = cell.step_with_jacobian(state, None, wx=wx)
    jb = torch.randn(2, 37, 4, 4, 8, generator=g) * 0.6
    rb = torch.randn(2, 37, 4, 8, generator=g)
    db = scan_block4(jb, rb)
    jd = torch.randn(2, 19, 6, 6, generator=g) * 0.4
    rd = torch.randn(2, 19, 6, generator=g)
    dd = scan_dense(jd, rd)
    pre = torch.randn(2, 300, 4 * 8, generator=g) * 2.0
    h0 = torch.randn(2, 4, 8, generator=g)
    h0[:, 1] = h0[:, 1].abs()
    fg = slstm_frozen_gate_scan_eager(pre, eps=1e-6, h0=h0)
    fg0 = slstm_frozen_gate_scan_eager(pre, eps=1e-6, h0=None)
    torch.manual_seed(99)
    gcell = ParaGRU(8, 2 * 64, mix="head", n_heads=2)
    hp = torch.randn(3, 4, 128, generator=g) * 0.5
    gwx = torch.randn(3, 4, 3 * 128, generator=g)
    with torch.no_grad():
        gnew, gjac = gcell.step_with_jacobian(hp, None, wx=gwx)
    _save(
        "parts",
        dict(
            slstm_R=cell.R, slstm_state=state, slstm_wx=wx, slstm_new=new, slstm_jac=jac,
            scan4_j=jb, scan4_r=rb, scan4_out=db, scand_j=jd, scand_r=rd, scand_out=dd,
            fg_pre=pre, fg_h0=h0, fg_out=fg, fg_out_noh0=fg0,
            gru_A_z=gcell.A_z, gru_A_r=gcell.A_r, gru_A_n=gcell.A_n, gru_h=hp, gru_wx=gwx,
            gru_new=gnew, gru_jac=gjac,
        ),
        dict(eps=1e-6),
    )


def slstm_bwd_case(name, *, d_in, d, B, T, K, P, dtype, seed, with_h0=False):
    """Gradients of sum(g * H) through newton_apply's eq. 2.6 backward."""
    from pararnn import ParaSLSTM, newton_apply, sequential_apply

    torch.manual_seed(seed)
    cell = ParaSLSTM(d_in, d, mix="diag").to(dtype)
    gen = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(B, T, d_in, generator=gen).to(dtype)
    grad = torch.randn(B, T, 4, d, generator=gen).to(dtype)
    tensors = {}
    h0 = None
    if with_h0:
        xp = torch.randn(B, 16, d_in, generator=gen).to(dtype)
        with torch.no_grad():
            h0 = sequential_apply(cell, xp)[:, -1].clone()
        tensors["h0"] = h0.clone()
        h0 = h0.requires_grad_(True)
    xg = x.clone().requires_grad_(True)
    H = newton_apply(cell, xg, _cfg(K, P), h0=h0)
    (H.float() * grad.float()).sum().backward()
    tensors.update(
        x=x, W=cell.W_x.weight.detach(), b=cell.W_x.bias.detach(), R=cell.R.detach(),
        grad=grad, newton=H.detach(),
        grad_x=xg.grad, grad_W=cell.W_x.weight.grad, grad_b=cell.W_x.bias.grad,
        grad_R=cell.R.grad,
    )
    if with_h0:
        tensors["grad_h0"] = h0.grad
    meta = dict(cell="ParaSLSTM", mix="diag", d_in=d_in, d=d, B=B, T=T, K=K, P=P,
                dtype=str(dtype).replace("torch.", ""), seed=seed, eps=cell.eps,
                max_recurrent_norm=cell.max_recurrent_norm, h0=with_h0,
                loss="sum(grad.float() * H.float())")
    _save(name, tensors, meta)


def bwd_parts_case():
    """The reverse 4x4 scan and the packed sLSTM cell VJP on random operands."""
    from pararnn.kernels.vjp_slstm import slstm_recurrence_vjp_eager
    from pararnn.solvers.scan import reverse_scan_block4

    g = torch.Generator().manual_seed(4321)
    jb = torch.randn(2, 41, 4, 4, 8, generator=g) * 0.6
    pb = torch.randn(2, 41, 4, 8, generator=g)
    mu = reverse_scan_block4(jb, pb)
    state = torch.randn(2, 33, 4, 16, generator=g)
    state[..., 1, :] = state[..., 1, :].abs() + 0.1
    wx = torch.randn(2, 33, 64, generator=g)
    r = torch.randn(4, 16, generator=g) * 0.3
    vmu = torch.randn(2, 33, 4, 16, generator=g)
    g_wx, g_r = slstm_recurrence_vjp_eager(state, wx, r, vmu, 1e-6)
    _save(
        "bwd_parts",
        dict(rev4_j=jb, rev4_p=pb, rev4_mu=mu, vjp_state=state, vjp_wx=wx, vjp_r=r, vjp_mu=vmu,
             vjp_gwx=g_wx, vjp_gr=g_r),
        dict(eps=1e-6),
    )


def gru_head_bwd_case(name, *, d_in, d, n_heads, B, T, K, dtype, seed, with_h0=False):
    """Gradients of sum(g * H) through newton_apply's eq. 2.6 backward (head GRU)."""
    from pararnn import ParaGRU, newton_apply

    torch.manual_seed(seed)
    cell = ParaGRU(d_in, d, mix="head", n_heads=n_heads).to(dtype)
    gen = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(B, T, d_in, generator=gen).to(dtype)
    grad = torch.randn(B, T, d, generator=gen).to(dtype)
    tensors = {}
    h0 = None
    if with_h0:
        h0 = (0.5 * torch.randn(B, d, generator=gen)).to(dtype)
        tensors["h0"] = h0.clone()
        h0 = h0.requires_grad_(True)
    xg = x.clone().requires_grad_(True)
    H = newton_apply(cell, xg, _cfg(K, None), h0=h0)
    (H.float() * grad.float()).sum().backward()
    tensors.update(
        x=x, W=cell.W_x.weight.detach(), b=cell.W_x.bias.detach(), A_z=cell.A_z.detach(),
        A_r=cell.A_r.detach(), A_n=cell.A_n.detach(), grad=grad, newton=H.detach(),
        grad_x=xg.grad, grad_W=cell.W_x.weight.grad, grad_b=cell.W_x.bias.grad,
        grad_A_z=cell.A_z.grad, grad_A_r=cell.A_r.grad, grad_A_n=cell.A_n.grad,
    )
    if with_h0:
        tensors["grad_h0"] = h0.grad
    meta = dict(cell="ParaGRU", mix="head", d_in=d_in, d=d, n_heads=n_heads, B=B, T=T, K=K,
                dtype=str(dtype).replace("torch.", ""), seed=seed,
                max_recurrent_norm=cell.max_recurrent_norm, h0=with_h0,
                loss="sum(grad.float() * H.float())")
    _save(name, tensors, meta)


def gru_head_bwd_parts_case():
    """The factorised head J^T mu and the eager head cell VJP on random operands."""
    from pararnn.kernels.gru_head_factor import gru_head_jt_mvp
    from pararnn.kernels.vjp_gru import gru_head_recurrence_vjp_eager

    g = torch.Generator().manual_seed(2468)
    hh, dh = 2, 64
    a = [torch.randn(hh, dh, dh, generator=g) * 0.2 for _ in range(3)]
    h = torch.randn(3, 5, hh, dh, generator=g) * 0.6
    z, r, n = (torch.rand(3, 5, hh, dh, generator=g) for _ in range(3))
    n = 2 * n - 1
    mu = torch.randn(3, 5, hh, dh, generator=g)
    jt = gru_head_jt_mvp(h, z, r, n, a[0], a[1], a[2], mu)
    hp = torch.randn(2, 9, hh * dh, generator=g) * 0.6
    wx = torch.randn(2, 9, 3 * hh * dh, generator=g)
    vmu = torch.randn(2, 9, hh * dh, generator=g)
    g_wx, g_az, g_ar, g_an = gru_head_recurrence_vjp_eager(hp, wx, a[0], a[1], a[2], vmu,
                                                           n_heads=hh, d_head=dh)
    _save(
        "gru_head_bwd_parts",
        dict(a_z=a[0], a_r=a[1], a_n=a[2], jt_h=h, jt_z=z, jt_r=r, jt_n=n, jt_mu=mu, jt_out=jt,
             vjp_h=hp, vjp_wx=wx, vjp_mu=vmu, vjp_gwx=g_wx, vjp_gaz=g_az, vjp_gar=g_ar,
             vjp_gan=g_an),
        dict(n_heads=hh, d_head=dh),
    )


def para_rnn_case(name, cell_kind, *, d_in, d, layers, B, T, K, P, seed, n_heads=None):
    """A stacked ParaRNN: Newton forward in train(), sequential in eval(), with the
    state_dict so a model can be loaded by parameter name."""
    from pararnn import NewtonConfig, ParaGRU, ParaRNN, ParaSLSTM

    torch.manual_seed(seed)
    if cell_kind == "slstm":
        cell = ParaSLSTM(d_in, d, mix="diag")
    else:
        cell = ParaGRU(d_in, d, mix="head", n_heads=n_heads)
    cfg = NewtonConfig(max_iters=K, residual_atol=None, residual_fail=None, picard_iters=P,
                       picard_adapt=False, scan_backend="eager")
    model = ParaRNN(cell, num_layers=layers, config=cfg, return_hidden=True)
    gen = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(B, T, d_in, generator=gen)
    with torch.no_grad():
        model.train()
        y_newton, last_newton = model(x)
        model.eval()
        y_seq, last_seq = model(x)
    tensors = {f"sd.{k}": v for k, v in model.state_dict().items()}
    tensors.update(x=x, y_newton=y_newton, last_newton=last_newton, y_seq=y_seq, last_seq=last_seq)
    meta = dict(cell=cell_kind, d_in=d_in, d=d, layers=layers, B=B, T=T, K=K, P=P, seed=seed,
                n_heads=n_heads)
    _save(name, tensors, meta)


def ragged_case(name, cell_kind, *, d_in, d, lengths, K, P, seed, n_heads=None):
    """Packed sequences: newton_apply and sequential_apply with cu_seqlens and
    per-sequence h0 (eager backend)."""
    from pararnn import ParaGRU, ParaSLSTM, newton_apply, sequential_apply

    torch.manual_seed(seed)
    if cell_kind == "slstm":
        cell = ParaSLSTM(d_in, d, mix="diag")
    else:
        cell = ParaGRU(d_in, d, mix="head", n_heads=n_heads)
    gen = torch.Generator().manual_seed(seed + 1)
    n = sum(lengths)
    cs = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0).tolist()), dtype=torch.long)
    x = torch.randn(1, n, d_in, generator=gen)
    if cell_kind == "slstm":
        xp = torch.randn(len(lengths), 16, d_in, generator=gen)
        with torch.no_grad():
            h0 = sequential_apply(cell, xp)[:, -1].clone()
    else:
        h0 = 0.5 * torch.randn(len(lengths), d, generator=gen)
    with torch.no_grad():
        H = newton_apply(cell, x, _cfg(K, P), h0=h0, cu_seqlens=cs)
        Hs = sequential_apply(cell, x, h0, cu_seqlens=cs)
    tensors = dict(x=x, h0=h0, cu_seqlens=cs, newton=H, sequential=Hs,
                   W=cell.W_x.weight, b=cell.W_x.bias)
    if cell_kind == "slstm":
        tensors["R"] = cell.R
    else:
        tensors.update(A_z=cell.A_z, A_r=cell.A_r, A_n=cell.A_n)
    meta = dict(cell=cell_kind, d_in=d_in, d=d, lengths=list(lengths), K=K, P=P, seed=seed,
                n_heads=n_heads, eps=getattr(cell, "eps", None),
                max_recurrent_norm=cell.max_recurrent_norm)
    _save(name, tensors, meta)


def auto_picard_table():
    from pararnn.solvers.newton.picard import slstm_auto_picard

    return {str(t): slstm_auto_picard(t) for t in (1, 64, 65, 2048, 2049, 16384, 131072)}


CASES = {
    "parts": parts_case,
    # BASELINE config 1, the reference's CPU-runnable parity case.
    "slstm_cfg1_fp32": lambda: slstm_case(
        "slstm_cfg1_fp32", d_in=64, d=64, B=2, T=1024, K=2, P=3, dtype=torch.float32, seed=0,
        keep_wx=False),
    "slstm_h0_fp32": lambda: slstm_case(
        "slstm_h0_fp32", d_in=24, d=32, B=2, T=200, K=3, P=1, dtype=torch.float32, seed=5,
        with_h0=True),
    "slstm_bf16": lambda: slstm_case(
        "slstm_bf16", d_in=64, d=64, B=2, T=512, K=2, P=3, dtype=torch.bfloat16, seed=1),
    "slstm_fp16": lambda: slstm_case(
        "slstm_fp16", d_in=64, d=64, B=2, T=512, K=2, P=3, dtype=torch.float16, seed=13,
        with_h0=True),
    "slstm_long_fp32": lambda: slstm_case(
        "slstm_long_fp32", d_in=16, d=16, B=1, T=4096, K=2, P=5, dtype=torch.float32, seed=2,
        x_std=0.5),
    "gru_head_fp32": lambda: gru_head_case(
        "gru_head_fp32", d_in=64, n_heads=2, d_head=64, B=2, T=256, K=3, dtype=torch.float32,
        seed=3),
    "gru_head_h0_fp32": lambda: gru_head_case(
        "gru_head_h0_fp32", d_in=32, n_heads=2, d_head=64, B=1, T=96, K=3, dtype=torch.float32,
        seed=4, with_h0=True),
    "gru_head_bf16": lambda: gru_head_case(
        "gru_head_bf16", d_in=64, n_heads=2, d_head=64, B=1, T=128, K=3, dtype=torch.bfloat16,
        seed=6),
    "gru_head_fp16": lambda: gru_head_case(
        "gru_head_fp16", d_in=64, n_heads=2, d_head=64, B=2, T=128, K=3, dtype=torch.float16,
        seed=14, with_h0=True),
    "bwd_parts": bwd_parts_case,
    "slstm_bwd_fp32": lambda: slstm_bwd_case(
        "slstm_bwd_fp32", d_in=24, d=32, B=2, T=256, K=3, P=3, dtype=torch.float32, seed=7,
        with_h0=True),
    "slstm_bwd_bf16": lambda: slstm_bwd_case(
        "slstm_bwd_bf16", d_in=32, d=32, B=2, T=256, K=2, P=3, dtype=torch.bfloat16, seed=8),
    "slstm_bwd_fp16": lambda: slstm_bwd_case(
        "slstm_bwd_fp16", d_in=32, d=32, B=2, T=256, K=2, P=3, dtype=torch.float16, seed=15),
    "slstm_ragged_fp32": lambda: ragged_case(
        "slstm_ragged_fp32", "slstm", d_in=12, d=16, lengths=(37, 100, 64), K=2, P=3, seed=11),
    "gru_head_ragged_fp32": lambda: ragged_case(
        "gru_head_ragged_fp32", "gru_head", d_in=16, d=128, lengths=(20, 45, 7), K=3, P=None,
        seed=12, n_heads=2),
    "gru_head_bwd_fp32": lambda: gru_head_bwd_case(
        "gru_head_bwd_fp32", d_in=16, d=128, n_heads=2, B=2, T=80, K=3, dtype=torch.float32,
        seed=31, with_h0=True),
    "gru_head_bwd_bf16": lambda: gru_head_bwd_case(
        "gru_head_bwd_bf16", d_in=16, d=128, n_heads=2, B=2, T=64, K=3, dtype=torch.bfloat16,
        seed=32),
    "gru_head_bwd_fp16": lambda: gru_head_bwd_case(
        "gru_head_bwd_fp16", d_in=16, d=128, n_heads=2, B=2, T=64, K=3, dtype=torch.float16,
        seed=33),
    "gru_head_bwd_parts": gru_head_bwd_parts_case,
    "para_rnn_slstm_fp32": lambda: para_rnn_case(
        "para_rnn_slstm_fp32", "slstm", d_in=12, d=32, layers=2, B=2, T=60, K=3, P=3, seed=41),
    "para_rnn_gru_head_fp32": lambda: para_rnn_case(
        "para_rnn_gru_head_fp32", "gru_head", d_in=12, d=128, layers=2, B=2, T=50, K=3, P=None,
        seed=42, n_heads=2),
}


def main(argv: list[str]) -> int:
    """Write every fixture, or only the cases named on the command line."""
    torch.set_num_threads(8)
    names = argv or list(CASES)
    unknown = [n for n in names if n not in CASES]
    if unknown:
        raise SystemExit(f"unknown cases {unknown}; known: {sorted(CASES)}")
    for n in names:
        CASES[n]()
    if not argv:
        with open(os.path.join(HERE, "auto_picard.json"), "w") as f:
            json.dump(auto_picard_table(), f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
