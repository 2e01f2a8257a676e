import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

SEED = 0xAFFE  # the reference tests' seed (tests/tensor/test_tensor_layout.py:34)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import torch_spyre_amd  # noqa: F401  (loads libspyre_hip.so; raises if not built)

    return torch.device("cuda", 0)
