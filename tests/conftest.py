import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# GEV2_PKG_ROOT: another directory holding graph_executor_v2 (the sanitizer
# build of the binding modules); the in-tree package otherwise
PKG_ROOT = os.environ.get("GEV2_PKG_ROOT") or os.path.join(REPO, "ai_framework-dev_amd")
for p in (REPO, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libgev2.so on the device)")


@pytest.fixture(scope="session")
def gpu():
    """The C-ABI library with a visible device; a GPU test without one fails loudly."""
    from graph_executor_v2.ops import capi

    capi.lib()
    if capi.device_count() < 1:
        pytest.fail("no HIP device visible to libgev2.so")
    return capi
