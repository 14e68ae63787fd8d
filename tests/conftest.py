import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("mini-inference-engine_amd", "oracle"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    import torch

    from minillm_amd import mi355x_fp8

    if not mi355x_fp8.mi355x_available():
        pytest.fail("gpu-marked test run without a gfx950 GPU")
    return torch.device("cuda:0")
