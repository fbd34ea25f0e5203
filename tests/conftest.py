import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "historic-htr-ocr_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu where one is present")


@pytest.fixture(scope="session")
def dev():
    import htr

    d = htr.Device(0)
    name, n_cu = d.info()
    print(f"\n[device] {name}, {n_cu} CUs", flush=True)
    yield d
    d.close()
