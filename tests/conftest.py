import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session", autouse=True)
def _built():
    """Build the HIP library and the oracle only if they are not built yet."""
    from mlxr_amd import qgemm
    if not os.path.exists(qgemm.LIB_PATH):
        from mlxr_amd import build
        build.build()
    from oracle import orc
    if not os.path.exists(orc.LIB_PATH):
        from oracle import build as obuild
        obuild.build()
    yield


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
