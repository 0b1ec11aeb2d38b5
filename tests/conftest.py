import os
import sys
from pathlib import Path

# torch's CPU kernels as the reference's platform (an AVX2 desktop CPU) runs
# them; the decode fixtures were written with them.  Must precede the first
# import of torch.
os.environ.setdefault("ATEN_CPU_CAPABILITY", "avx2")

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def torch_cpu_like_fixture():
    """torch with the AVX2 CPU kernels and oneDNN off, as the fixtures were
    written; skips when torch was imported with other kernels."""
    import torch
    torch.backends.mkldnn.enabled = False
    if torch.backends.cpu.get_cpu_capability() != "AVX2":
        pytest.skip("torch CPU kernels are not the AVX2 ones (imported before conftest)")
    return torch


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return torch.device("cuda:0")
