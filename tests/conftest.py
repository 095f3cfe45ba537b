import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def pkg():
    """The package (kaggle-llm-endpoint_amd/) imported as kaggle_llm_endpoint_amd."""
    import __graft_entry__ as ge
    return ge.load_package()


@pytest.fixture(scope="session")
def gpu(pkg):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg._lib.lib()          # fails loudly if the HIP library is not built
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def full_cb3_layer(pkg, gpu):
    """Three CB3 experts at the benchmark's matrix shapes (hidden 6144, intermediate 2048) with the oracle's view of
    them, built once per session (generating canonical codes on the host takes tens of seconds)."""
    import numpy as np
    from tests.util import Layer
    L = Layer(np.random.default_rng(2026), "CB3", 3, 6144, 2048)
    return L, L.tables(pkg)
