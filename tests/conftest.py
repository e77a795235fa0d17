from pathlib import Path
import sys

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT / "cuda-moe-engine_amd", ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    import torch

    torch.set_num_threads(1)
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def gpu_available():
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def ext():
    from moe_dispatch._extension import get_extension

    return get_extension()
