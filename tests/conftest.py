import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "mlx-runner_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through libmlxr's C ABI")


@pytest.fixture(scope="session")
def gpu():
    import mlxr
    assert mlxr.device_count() > 0, "no GPU visible: GPU tests must run on the MI355X box"
    return mlxr
