import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    # The oracle and the library are built by __graft_entry__.build(); build
    # them here too when missing so a fresh checkout can run the CPU suite.
    if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True,
                       stdout=subprocess.DEVNULL)
    lib = os.path.join(ROOT, "cosxamix_amd", "lib", "libcosxamix_hip.so")
    if not os.path.exists(lib) and os.path.exists("/opt/rocm/bin/hipcc"):
        from cosxamix_amd import build
        build.build()


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    return O


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    return np.load(os.path.join(ROOT, "tests", "golden", "kquant_rows.npz"))


@pytest.fixture(scope="session")
def dev():
    """The GPU; GPU tests fail (they do not skip) when there is none."""
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch.device("cuda:0")
