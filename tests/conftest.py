import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def has_gpu_device() -> bool:
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def gpu():
    """The torch module with the GPU initialised; GPU tests fail (not fall back)
    when the device nodes exist but HIP does not come up."""
    if not has_gpu_device():
        pytest.skip("no GPU device in this container")
    import torch

    assert torch.cuda.is_available(), "GPU device present but torch.cuda is not available"
    torch.cuda.init()
    return torch


def norm_rel(a, b) -> float:
    """max|a - b| / max|b|: the norm-relative error used for every parity bar."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.abs(b).max()
    if den == 0:
        return float(np.abs(a).max())
    return float(np.abs(a - b).max() / den)


def bf16_round(x):
    """Round an fp32/fp64 numpy array to bf16 precision (nearest even), as fp32."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)
