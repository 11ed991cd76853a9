import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Skip-free guard: GPU tests are selected with -m gpu; fail loudly if no GPU is visible."""
    if not _gpu_available():
        pytest.fail("GPU test selected but torch.cuda.is_available() is False")
    import torch

    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def qhtp_lib():
    """The built libqhtp.so (built on demand if absent, e.g. in a fresh CPU checkout)."""
    from qcom_htp_amd import _lib

    if not _lib.LIB_PATH.exists():
        from qcom_htp_amd.build import build

        build(verbose=False)
    return _lib.lib()
