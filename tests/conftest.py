import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    # the kernel-choice table reads its tuning file on first use: the tests get
    # an empty directory of their own, never a user's tuned choices
    import tempfile

    os.environ["TORCHVULKAN_CACHE_DIR"] = tempfile.mkdtemp(prefix="tvk-tuning-")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Skips GPU tests when no GPU is visible; fails loudly if the HIP library is missing."""
    if not _gpu_available():
        pytest.skip("no GPU visible")
    from torchvulkan_amd import _abi

    _abi.load()  # raises when libtvk_hip.so is not built: never a silent fallback
    return _abi
