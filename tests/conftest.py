import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def backend():
    """One desk for the whole GPU session (one process, one stream)."""
    from igllm_amd.backend import Backend

    b = Backend(device=0, sum_limit=1024, col_limit=16384, lane_limit=16)
    yield b
    b.close()


@pytest.fixture(scope="session")
def ref_plain():
    import oracle_lib

    lib = oracle_lib.ref("plain")
    if lib is None:
        pytest.skip("oracle/_ref was not built (reference source absent when build() ran)")
    return lib
