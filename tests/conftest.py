import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "fpga-llama-gguf_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); runs the kernels through the C ABI")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def gq():
    import gemvq

    return gemvq


@pytest.fixture(scope="session")
def orc():
    import oracle

    if not os.path.exists(oracle.ORC_PATH):  # a fresh checkout: the oracle builds in seconds
        oracle.build(ref=False)
    return oracle
