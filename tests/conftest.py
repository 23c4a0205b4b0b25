import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import sv_oracle
    sv_oracle.lib()
    return sv_oracle


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with the extension loaded; a GPU test fails (not skips) without one."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    import eccv26_tad_amd  # noqa: F401

    return torch.device("cuda:0")
