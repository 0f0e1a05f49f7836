import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The device handle. A missing device skips; a missing or broken library
    fails (the reference's rule, crates/llmtie-cuda/tests/kernels.rs:103-119:
    an absent GPU is an environment fact, a build failure is a defect)."""
    import torch
    from ttsxabe_amd import _lib
    _lib.lib()  # raises if not built
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from ttsxabe_amd.gpu import Gpu
    return Gpu(int(os.environ.get("LLMTIE_TEST_DEVICE", "0")))
