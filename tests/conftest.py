import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "cohere-transcribe_amd"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP backend)")
    config.addinivalue_line("markers", "slow: long CPU oracle runs")


@pytest.fixture(scope="session")
def kernel_model():
    import ctbind as cb
    return cb.SynthModel(seed=11, variant=1)


@pytest.fixture(scope="session")
def hip():
    """libct_hip.so with backend_init(0) done once for the test process."""
    import ctbind as cb
    lib = cb.hip()
    if lib.backend_num_devices() < 1:
        pytest.fail("no HIP device visible")
    lib.backend_init(0)
    return lib
