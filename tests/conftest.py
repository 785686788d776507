import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "dtree-mlx_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libdtree_hip.so")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from dtree_hip import _native

    _native.lib()  # fail loudly if the native library is missing
    return torch.device("cuda:0")


@pytest.fixture(params=["head", "group"])
def attn_kernel(request, monkeypatch):
    """Both tree-attention designs (per query head, per KV group); the library
    picks one by the prefix its grid is sized for, DTREE_ATTN_KERNEL forces it
    here (read at every launch)."""
    monkeypatch.setenv("DTREE_ATTN_KERNEL", request.param)
    return request.param
