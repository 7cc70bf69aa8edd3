import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libwhisper_hip.so on the device)")


@pytest.fixture(scope="session")
def wh():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    return oracle


@pytest.fixture(scope="session")
def gpu(wh):
    # torch is never imported next to libwhisper_hip.so: it bundles its own
    # HIP runtime and a second copy in the process would be loaded
    if wh.native.device_count() < 1:
        pytest.skip("no GPU visible")
    return 0


def rel_err(got, want):
    """max |got - want| / max |want|: the logits tolerance metric (1e-3)."""
    import numpy as np

    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))
