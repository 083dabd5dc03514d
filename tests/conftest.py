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
