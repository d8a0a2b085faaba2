import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "llmtoy-zig_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def ctx():
    import llmtoy_amd as lt
    c = lt.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="session")
def pool():
    import pyoracle as orc
    p = orc.Pool(min(16, os.cpu_count() or 1))
    yield p
    p.close()
