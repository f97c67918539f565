import os
import sys

# torch first: the HIP kernels must bind to the HIP runtime torch loads.
import torch  # noqa: F401
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def gpu():
    """GPU tests fail (not skip) without a GPU: they are run only on the GPU box."""
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    import vkwr  # noqa: F401  (loads the extension modules; raises if absent)
    return torch.device("cuda:0")
