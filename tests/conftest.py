import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_runtest_setup(item):
    # Name the case before any GPU work so a crash log identifies it.
    if item.get_closest_marker("gpu") is not None:
        sys.stdout.write(f"\n[gpu-case] {item.nodeid}\n")
        sys.stdout.flush()


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    from intent_amd import _native

    arch = _native.device_arch(0)
    assert arch.split(":")[0] == "gfx950", f"expected gfx950, found {arch}"
    torch.backends.cuda.matmul.allow_tf32 = False
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def threads():
    return max(1, min(16, len(os.sched_getaffinity(0))))
