import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "dw-tpu_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from dw_tpu_amd import _lib
    _lib.load()  # a missing library where a GPU is present is a failure, not a skip
    return torch.device("cuda:0")


@pytest.fixture
def rng():
    return np.random.Generator(np.random.PCG64(20261201))


def bf16_tensor(bits, device):
    """uint16 bf16 bit patterns (numpy) -> torch bf16 tensor on device."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_bits(t):
    """torch bf16 tensor -> uint16 numpy bit patterns."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
