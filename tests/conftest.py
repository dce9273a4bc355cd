import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path through the C ABI)")


def _gpu_present() -> bool:
    try:
        import tierstream_amd as tsa
        return tsa.gpu_count() > 0
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """The HIP path on device 0. A GPU test fails (never skips to a fallback) when the library is missing."""
    import tierstream_amd as tsa
    tsa.lib()  # raises if the product library is not built
    if tsa.gpu_count() == 0:
        pytest.fail("no HIP device visible to a test marked gpu")
    tsa.check(tsa.lib().tsa_set_device(0))
    return tsa


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.olib()
    return o


def pytest_report_header(config):
    return f"tierstream_amd tests, root {ROOT}, HIP_VISIBLE_DEVICES={os.environ.get('HIP_VISIBLE_DEVICES')}"
