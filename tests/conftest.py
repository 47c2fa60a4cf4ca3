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


def pytest_sessionfinish(session, exitstatus):
    """Write every parity check's metrics to $SOKLYN_PARITY_REPORT (JSON lines), when set."""
    path = os.environ.get("SOKLYN_PARITY_REPORT")
    if not path:
        return
    import json
    from tests import helpers
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as f:
        for r in helpers.RECORDS:
            f.write(json.dumps(r) + "\n")
