import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "kimi-k3-in-rust_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU")


def _ensure_built():
    import __graft_entry__ as g
    g._ensure_built()


_ensure_built()


@pytest.fixture(scope="session")
def gpu():
    import k3moe
    if k3moe.gpu_count() < 1:
        pytest.skip("no GPU visible")
    return k3moe
