import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "jero-kernels-rvv_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP library")


@pytest.fixture(scope="session")
def gpu():
    """Initializes device 0 for the GPU tier; the product library must be built."""
    import torch

    import jk

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    jk.lib()  # raises if libjk.so is missing: no fallback path exists
    jk.init(0)
    jk.host_cache_set_limit(4 << 30)  # the host tier's resident weights, across the whole session
    torch.cuda.init()
    return torch
