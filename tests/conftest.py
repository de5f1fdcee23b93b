import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950); run with -m gpu")


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle
    return pyoracle.get()


@pytest.fixture(scope="session")
def gpu():
    """The torch module with a usable gfx950 device and libhipgemm loaded."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import hipgemm_amd
    hipgemm_amd.lib()  # raises if the native library is missing
    name = torch.cuda.get_device_properties(0).gcnArchName
    assert "gfx950" in name, f"expected gfx950, found {name}"
    return torch
