import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libsoklyn_hip.so")


@pytest.fixture(scope="session")
def ctx():
    import torch
    from soklyn_amd import abi
    # An explicit (default-priority) stream: torch's legacy default stream has handle 0,
    # which the C ABI would read as "use the context's own stream".
    s = torch.cuda.Stream()
    torch.cuda.set_stream(s)
    c = abi.Context(0, 16)
    c.set_stream(s.cuda_stream)
    yield c
    torch.cuda.synchronize()
    c.close()
