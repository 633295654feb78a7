"""Test configuration: import paths, the ``gpu`` marker and shared helpers."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (os.path.join(ROOT, "ayaka-py_amd"), ROOT):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from ayaka.kernel.hip import _lib

    lib = _lib.load_library()
    assert lib.ayk_device_supported(0) == 1, "device 0 is not gfx950"
    return torch.device("cuda:0")
