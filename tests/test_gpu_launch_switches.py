"""The launch-per-pass / launch-per-iteration fallbacks of the sLSTM solve
(PRNN_SLSTM_PICARD_FUSED=0, PRNN_SLSTM_NEWTON_FUSED=0: read once per
process by the library, so they run in a child process) against the default
single-launch path on the same inputs: same algebra, other scan association
and launch boundaries, so they agree to rounding.  Every case prints its name
before running."""

import os
import subprocess
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

_CHILD = r"""
import sys
sys.path[:0] = [{pkg!r}, {repo!r}]
import torch
from pararnn_amd import NewtonConfig, ParaSLSTM, newton_apply
torch.manual_seed(0)
cell = ParaSLSTM(32, 256).to("cuda:0", {dtype})
g = torch.Generator(device="cuda:0").manual_seed(1)
x = (torch.randn(2, 3000, 32, generator=g, device="cuda:0") * 0.5).to({dtype})
cfg = NewtonConfig(max_iters=3, picard_iters=3, residual_atol=None, residual_fail=None,
                   picard_adapt=False)
torch.use_deterministic_algorithms(True, warn_only=True)
with torch.no_grad():
    out = newton_apply(cell, x, cfg)
torch.save(out.cpu(), {path!r})
"""


def _run(tmp_path, tag, dtype, env):
    path = str(tmp_path / f"{tag}.pt")
    code = _CHILD.format(pkg=os.path.join(REPO, "pararnn-torch_amd"), repo=REPO,
                         dtype=dtype, path=path)
    full = dict(os.environ)
    full.update(env)
    subprocess.run([sys.executable, "-c", code], env=full, check=True, timeout=300)
    return torch.load(path, weights_only=True)


@pytest.mark.parametrize("dtype", ["torch.float32", "torch.bfloat16"])
def test_per_launch_fallbacks_match_single_launch(tmp_path, dtype):
    print(f"case launch switches {dtype}: fused vs PICARD_FUSED=0 NEWTON_FUSED=0", flush=True)
    fused = _run(tmp_path, "fused", dtype, {})
    split = _run(tmp_path, "split", dtype,
                 {"PRNN_SLSTM_PICARD_FUSED": "0", "PRNN_SLSTM_NEWTON_FUSED": "0"})
    assert fused.shape == split.shape and torch.isfinite(fused).all()
    rel = ((fused.float() - split.float()).abs() / (1 + fused.float().abs())).max().item()
    print(f"  max rel diff {rel:.2e}", flush=True)
    # bf16: a few storage ulps (fp32 scans associated differently, then
    # rounded to bf16)
    assert rel <= (1e-5 if dtype == "torch.float32" else 2 ** -6)
