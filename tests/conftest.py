import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "qora-tts-12hz-1.7b_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libqtts_hip.so)")


def gpu_present():
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def ctx_factory():
    """Contexts on device 0.  Fails (does not skip) when a GPU is present but
    the HIP library is missing or broken: there is no fallback path."""
    if not gpu_present():
        pytest.skip("no GPU in this container")
    import qtts
    made = []

    def make(kv_capacity=4096):
        c = qtts.Context(0, kv_capacity=kv_capacity)
        made.append(c)
        return c

    yield make
    for c in made:
        c.close()
