import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")


@pytest.fixture(autouse=True)
def no_stalled_launches(request):
    """After every GPU test: no fused decode launch of the test had a cross-wave wait run out (a
    stalled launch completes with unreliable outputs; the library counts them per workspace)."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import torch
    if not torch.cuda.is_available():
        return
    from mlxlr8_amd._lib import stalled_launches
    torch.cuda.synchronize()
    n = stalled_launches()
    assert n == 0, f"{n} fused decode launch(es) had a bounded wait run out"


@pytest.fixture(scope="session")
def orc():
    from oracle import lib
    return lib()


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import mlxlr8_amd
    mlxlr8_amd.lib()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")


def bf16_bits(t):
    """torch bf16 tensor -> numpy uint16 bit patterns."""
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def f16_bits(t):
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def bits_to_f32(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
