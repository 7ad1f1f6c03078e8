import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
if str(ROOT / "tests") not in sys.path:
    sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built library")


@pytest.fixture(scope="session")
def stock():
    import oracle
    return oracle.stock()


@pytest.fixture(scope="session")
def ref():
    import oracle
    lib = oracle.ref()
    if lib is None:
        pytest.skip("oracle/_ref was not built (it needs /root/reference at build time)")
    return lib


@pytest.fixture(scope="session")
def hip():
    """The library with device 0 bound; skips nothing: a gpu test without a GPU is a failure."""
    import torch
    import burnisher_amd as bh
    assert torch.cuda.is_available(), "gpu test on a host without a GPU"
    lib = bh.lib()
    bh.check(lib.bh_init(0), "bh_init")
    return lib
