"""The W_x weight gradient gy^T x over B*T rows (split-K batched GEMM with fp32
partials on long reductions) against a float64 product."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.mark.parametrize("dtype,n,tol", [
    (torch.float32, 131072, 1e-5), (torch.float32, 65536 + 4096, 1e-5), (torch.float32, 5000, 1e-5),
    (torch.bfloat16, 131072, 1e-2), (torch.float32, 65539, 1e-5),
])
def test_weight_grad_matches_float64(dtype, n, tol):
    from pararnn_amd.newton import _weight_grad

    print(f"case weight grad {dtype} n={n}", flush=True)
    g = torch.Generator().manual_seed(n)
    gy = torch.randn(n, 384, generator=g).to(DEV, dtype)
    xx = torch.randn(n, 96, generator=g).to(DEV, dtype)
    got = _weight_grad(gy, xx)
    ref = gy.double().t() @ xx.double()
    rel = ((got.double() - ref).abs().max() / ref.abs().max()).item()
    print(f"  rel {rel:.2e}", flush=True)
    assert got.dtype == dtype and got.shape == (384, 96)
    assert rel <= tol
