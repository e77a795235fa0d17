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
    # The oracle's C checker (seconds to build with gcc) when build() has not made it yet.
    from oracle import moe_oracle

    if moe_oracle._C_GEMM is None:
        moe_oracle.build_c_checker()
        moe_oracle._C_GEMM = moe_oracle._load_c_gemm()
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def gpu_available():
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def ext():
    from moe_dispatch._extension import get_extension

    return get_extension()
