import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _no_expired_waits(request):
    """After every GPU test: no bounded LDS-flag wait of the library's kernels
    ran out (hipgpt_attn_wait_expired), i.e. no wave went on with data another
    wave had not yet published."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import torch

    if not torch.cuda.is_available():
        return
    from hipgpt_amd import _lib

    torch.cuda.synchronize()
    n = _lib.wait_expired(clear=True)
    assert n == 0, f"{n} bounded LDS-flag waits expired during this test"
