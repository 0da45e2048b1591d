import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import _util  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    return _util.load_oracle()


@pytest.fixture(scope="session")
def orc_omp():
    return _util.load_oracle(omp=True)


@pytest.fixture(scope="session")
def gen(orc):
    return _util.Gen(orc)


@pytest.fixture(scope="session")
def ref():
    r = _util.load_ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    return r


@pytest.fixture(scope="session")
def lib():
    """The product library on the GPU.  Fails (does not skip) if it is not built or
    the device cannot be opened: GPU tests must run the HIP path."""
    mod = _util.load_product()
    return mod.Lib().init()


@pytest.fixture(scope="session")
def torch_dev():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda:0")
