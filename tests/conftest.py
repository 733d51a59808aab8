import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def hip():
    """The C-ABI binding; GPU tests fail (not skip) if the library is missing."""
    from spar_amd import hip as binding

    binding.load()
    if binding.device_count() < 1:
        pytest.fail("no HIP device visible to a gpu-marked test")
    return binding


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    return oracle.lib()
