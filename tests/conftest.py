"""pytest configuration: import paths and the ``gpu`` marker.

Tests marked ``gpu`` need a MI355X (they launch libcascade_hip kernels);
everything else runs on a CPU-only host.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (os.path.join(ROOT, "cascade-llm_amd"), ROOT,
             os.path.join(ROOT, "tests")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a GPU (runs the libcascade_hip kernels)"
    )


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from layer_streaming import _hip

    _hip.load()
    return torch.device("cuda:0")
