import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    # load what is built; build only when nothing is (the GPU box runs prebuilt files)
    lib = os.path.join(ROOT, "libr3d_amd", "libr3d_gfx950.so")
    ora = os.path.join(ROOT, "oracle", "libr3d_oracle.so")
    if not (os.path.exists(lib) and os.path.exists(ora)):
        from libr3d_amd import build as B
        B.build_all()


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
