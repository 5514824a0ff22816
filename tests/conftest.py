import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "ming-tts_amd", "oracle", os.path.join("tests", "golden")):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


@pytest.fixture(scope="session")
def gpu():
    """The GPU test context: torch on cuda:0 and the loaded HIP library.  Fails (does not
    skip) without a GPU, so a GPU run can never pass on a fallback."""
    import torch

    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    import mingtts

    mingtts.load()
    torch.cuda.set_device(0)
    return torch.device("cuda", 0)
