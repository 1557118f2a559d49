import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# Before anything imports torch: the package loads its hipBLASLt ahead of PyTorch's own.
import dadgpt_amd  # noqa: E402,F401


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden_dir():
    return os.path.join(ROOT, "tests", "golden")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device. A GPU test fails (does not skip) when there is no GPU or the HIP
    library cannot be loaded: those tests only run where a GPU is expected."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    from dadgpt_amd import attention

    attention.lib()  # raises LibraryNotBuilt when missing
    name = torch.cuda.get_device_properties(0).gcnArchName
    print(f"[gpu] device 0: {name}", flush=True)
    return torch.device("cuda:0")
