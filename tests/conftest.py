import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "fhe-mamba_amd"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


import gc  # noqa: E402

import pytest  # noqa: E402


@pytest.fixture(autouse=True)
def _release_device_memory(request):
    """GPU tests build contexts whose keys and plaintext caches can take tens
    of GB; their objects reference each other, so collect the cycles after
    each test instead of letting several tests' device memory pile up."""
    yield
    if request.node.get_closest_marker("gpu") is not None:
        gc.collect()
