import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def hip():
    """The HIP device through libqvkv.  On a box without a GPU this fails loudly: GPU
    tests are selected with -m gpu only where a GPU exists."""
    import torch

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    torch.cuda.init()
    from qubivex_amd import HipDevice

    dev = HipDevice(0)
    print(f"device: {dev.describe()}", flush=True)
    yield dev
    dev.close()


@pytest.fixture
def knobs():
    """Sets launch-shape knobs through the library's qvkv_tune (knobs(name, value)); every
    knob is back at its default after the test."""
    from qubivex_amd import kv

    kv.tune_reset()
    yield kv.tune
    kv.tune_reset()
