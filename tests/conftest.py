import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parent.parent
for path in (REPO, REPO / "vllm-rlt_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm (gfx950) device; select with -m gpu")


def pytest_collection_modifyitems(config, items):
    gpu_items = [item for item in items if "gpu" in item.keywords]
    if gpu_items and not torch.cuda.is_available():
        skip = pytest.mark.skip(reason="no ROCm device visible")
        for item in gpu_items:
            item.add_marker(skip)


@pytest.fixture(autouse=True, scope="session")
def bounded_cpu_threads():
    # Same single-thread CPU policy as the reference suite (tests/conftest.py:22-27).
    previous = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(previous)
