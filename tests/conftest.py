import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")


@pytest.fixture
def no_stream_k():
    """One whole tile per block for every product (no stream-K): for checks
    that a row's bits do not depend on where the row lies, which the shared
    tiles of the stream-K schedule give up (they sum k in another order)."""
    from compact_amd import gemm
    gemm.set_stream_k(False)
    yield
    gemm.set_stream_k(True)
