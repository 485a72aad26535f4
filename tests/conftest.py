import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_sessionstart(session):
    # the CPU oracle is cheap to build; the GPU library is built by
    # __graft_entry__.build() (tests load what is there)
    orc = os.path.join(ROOT, "oracle", "liboracle.so")
    if not os.path.exists(orc):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "liboracle.so"], check=False)


@pytest.fixture(scope="session")
def tmpdir_s(tmp_path_factory):
    return tmp_path_factory.mktemp("sml")
