import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "fast-mario-env_amd"), os.path.join(ROOT, "tests"), os.path.join(ROOT, "tests", "golden"),
          os.path.join(ROOT, "tests", "golden", "roms")):
    if p not in sys.path:
        sys.path.insert(0, p)

# FME_TEST_SCALE multiplies frames / steps of the long differential tests (default 1).
SCALE = max(1, int(os.environ.get("FME_TEST_SCALE", "1")))


def scaled(n):
    return n * SCALE


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (runs the HIP library)")
    config.addinivalue_line("markers", "slow: long-running")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


HAVE_GPU = _gpu_available()
requires_gpu = pytest.mark.skipif(not HAVE_GPU, reason="no GPU")
