"""Shared test set-up: the `gpu` marker, import paths for the product binding (mako-image_amd/mkimage.py) and the
oracle (oracle/mkref.py), and fixtures."""
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT / "mako-image_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path through the C ABI)")


@pytest.fixture(scope="session")
def gpu():
    """The product library with a device; GPU tests fail loudly if the library is missing."""
    import mkimage

    lib = mkimage.lib()  # raises if libmkimage.so is not built
    n = mkimage.device_count()
    if n < 1:
        pytest.fail("no GPU visible to the HIP runtime")
    mkimage.call("mk_set_device", 0)
    # every GEMM / convolution / attention operand must lie inside a known allocation of the extent it needs
    mkimage.STRICT = True
    return mkimage


@pytest.fixture
def rng():
    return np.random.default_rng(0)
