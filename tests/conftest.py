"""Shared fixtures.  `gpu` tests need an MI355X; everything else runs on CPU."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    if not os.path.exists(O.lib_path()):
        O.build()
    return O


@pytest.fixture(scope="session")
def yl():
    import yallma3_mini_inference_amd as Y
    Y.lib()  # raises if the HIP library is not built
    return Y


@pytest.fixture(scope="session")
def gpu(yl):
    if yl.device_count() < 1:
        pytest.fail("no HIP device visible: gpu tests need an MI355X")
    return yl


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    d = os.environ.get("YL_MODEL_DIR")
    if d:
        os.makedirs(d, exist_ok=True)
        return d
    return str(tmp_path_factory.mktemp("models"))
