import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running check")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import phaseshift_amd
    phaseshift_amd.lib()   # fails loudly when the HIP library is missing
    return torch.device("cuda:0")


def pytest_runtest_logstart(nodeid, location):
    # name the case before it touches the GPU (flushed, so it survives a crash)
    import sys
    sys.stderr.write(f"\n[start] {nodeid}\n")
    sys.stderr.flush()
