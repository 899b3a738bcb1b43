import os
import sys

import pytest

REPO_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO_ROOT, "flash-attention_amd")
for p in (REPO_ROOT, PKG_DIR, os.path.join(REPO_ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (run with -m gpu)")
    config.addinivalue_line("markers", "slow: long-running test")


@pytest.fixture(scope="session")
def fa():
    """The product package (HIP path only; raises if the extension is absent)."""
    import flash_attention_runtime

    return flash_attention_runtime


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    return O
