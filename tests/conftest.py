import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)
GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "emu_jobs(*names): the CPU-emulation runs (tests/emu/jobs.py) a test reads")


def pytest_collection_modifyitems(config, items):
    names = set()
    for item in items:
        for mark in item.iter_markers("emu_jobs"):
            names.update(mark.args)
    if names:
        from tests.emu import jobs
        jobs.want(names)


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN
