import json
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "pararnn-torch_amd"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def load_golden(name: str):
    """(tensors, meta) of a committed fixture written by tests/golden/make_golden.py."""
    from safetensors import safe_open
    from safetensors.torch import load_file

    path = os.path.join(GOLDEN, f"{name}.safetensors")
    with safe_open(path, "pt") as f:
        meta = json.loads(f.metadata()["meta"])
    return load_file(path), meta


@pytest.fixture
def golden():
    return load_golden


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(params=[False, True], ids=["lookback_default", "lookback_deterministic"])
def lookback_mode(request):
    """Run a test with torch's deterministic-algorithms flag off and on: on,
    the sLSTM look-back scans take their deterministic walk, which must meet
    the same parity bar."""
    import torch

    prev = torch.are_deterministic_algorithms_enabled()
    prev_warn = torch.is_deterministic_algorithms_warn_only_enabled()
    torch.use_deterministic_algorithms(request.param, warn_only=True)
    yield request.param
    torch.use_deterministic_algorithms(prev, warn_only=prev_warn)
