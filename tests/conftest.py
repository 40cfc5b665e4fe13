import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT / "nano-vllm-diy_amd", ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (MI355X) and libpagedkv.so")


@pytest.fixture(scope="session")
def gpu():
    """The torch device for GPU tests; fails loudly if the GPU or the library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from pagedkv._lib import lib

    lib()  # raises if libpagedkv.so is not built: GPU tests never run without the kernels
    return torch.device("cuda:0")
