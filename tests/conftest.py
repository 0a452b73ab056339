import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); parity vs the oracle")
    config.addinivalue_line("markers", "slow: long-running (full-size composites)")


def has_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    if not has_gpu():
        pytest.skip("no HIP device")
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    return torch.device("cuda:0")


def announce(msg):
    """Flushes a line naming the case before a GPU step (so a hard failure
    still leaves the case name in the log)."""
    print(f"\n[case] {msg}", flush=True)
