import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built kernel library")


def _have_gpu() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture
def gpu():
    """Skip without a GPU; on a GPU box a missing library is a failure, not a skip."""
    if not _have_gpu():
        pytest.skip("no GPU visible to torch")
    from forgeml_amd import _native, kernels

    _native.load()  # raises NativeLibraryError when the library is not built
    import torch

    arch = kernels._device_arch(torch.device("cuda", 0))
    assert arch == kernels.TARGET_ARCH, f"GPU tests need {kernels.TARGET_ARCH}, found {arch}"
    return torch.device("cuda", 0)
