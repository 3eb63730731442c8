import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "ascendnpu-ir_amd"))
sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP kernels)")
    # the CPU restatement is test infrastructure; build it if this checkout lacks it
    if not os.path.exists(os.path.join(REPO, "oracle", "libhfref.so")):
        subprocess.run(["make", "-s", "-C", os.path.join(REPO, "oracle")], check=True)


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
