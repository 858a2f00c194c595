"""Test configuration: paths, the `gpu` marker, and shared fixtures.

`-m "not gpu"` runs on any CPU host: the oracle against the reference's
known answers and closed forms, the device-math emulation against the host
libm, and the C ABI's host-side checks. `-m gpu` needs an MI355X and compares
the HIP sampler with the oracle.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "oxide-tech-llm-engine_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); calls the sampler through its C ABI")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    return torch
