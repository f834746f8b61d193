import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _has_gpu():
    # no torch here: the library brings its own HIP runtime and device memory
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def gpu():
    if not _has_gpu():
        pytest.skip("no GPU")
    import pocketforge_amd as pf
    return pf.Context(0)


@pytest.fixture(scope="session")
def tiny_weights():
    from pocketforge_amd import weights as W
    return W.TINY, W.make_weights(W.TINY, seed=1234)


@pytest.fixture(scope="session")
def tiny_model(gpu, tiny_weights):
    import pocketforge_amd as pf
    cfg, w = tiny_weights
    return pf.Model(gpu, cfg, w)


@pytest.fixture()
def tiny_engine(tiny_model):
    import pocketforge_amd as pf
    e = pf.Engine(tiny_model, sink_size=4, window_size=64, pool_block=6, max_context=512)
    yield e
    e.close()
