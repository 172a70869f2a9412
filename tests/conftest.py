import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: full-size parity case (minutes of CPU oracle time)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import binding
    binding.lib()
    return binding


@pytest.fixture(scope="session")
def backend():
    """One HIP context for the whole GPU session; kernels run on torch's stream."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    from myelith_amd.backend import RocmBackend
    b = RocmBackend(0)
    b.use_torch_stream()
    yield b
    b.close()


@pytest.fixture(scope="session")
def luts64():
    from myelith_amd.luts import LutSet
    return LutSet.for_head_dim(64)


@pytest.fixture(scope="session")
def luts128():
    from myelith_amd.luts import LutSet
    return LutSet.for_head_dim(128)


def case(msg: str) -> None:
    """Names the case before a GPU step, flushed, so a crash still says what ran."""
    print(f"[case] {msg}", flush=True)
