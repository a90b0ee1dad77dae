import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """The HIP device 0 with the backend initialised (skips when no GPU)."""
    if not _gpu_available():
        pytest.skip("no GPU visible")
    import torch

    from c3_amd import native

    torch.cuda.init()
    native.init(0)
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def stream(gpu):
    import torch

    return torch.cuda.current_stream().cuda_stream


@pytest.fixture(autouse=True)
def _release_device_buffers():
    yield
    import sys as _sys

    mod = _sys.modules.get("tests.parity")
    if mod is not None:
        try:
            import torch

            if torch.cuda.is_available():
                torch.cuda.synchronize()
        except Exception:
            pass
        mod.release_buffers()
