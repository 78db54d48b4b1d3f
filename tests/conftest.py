import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs on the MI355X box)")


@pytest.fixture(scope="session")
def gpu():
    """The gfx950 device; GPU tests skip only where torch sees no GPU at all."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this container")
    dev = torch.device("cuda:0")
    arch = torch.cuda.get_device_properties(0).gcnArchName
    assert arch.startswith("gfx950"), f"the monokernels need gfx950, found {arch}"
    from sgl_amd_mono_amd import _lib

    _lib.lib()  # fails loudly when the HIP library is missing
    return dev
