import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "glm-flash-lite_amd")
ORACLE = os.path.join(ROOT, "oracle")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (runs the HIP path)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import REFLIB, RefEngine
    if not os.path.exists(REFLIB):
        pytest.skip("reference engine oracle/_ref/libftref.so not built")
    return RefEngine(threads=2, cpus=sorted(os.sched_getaffinity(0))[:2])


@pytest.fixture(scope="session")
def ref_server():
    """The reference engine built with its server's flags (default fp contraction), oracle/_ref/libftref_server.so."""
    from oracle import REFLIB_SERVER, RefEngine
    if not os.path.exists(REFLIB_SERVER):
        pytest.skip("reference engine oracle/_ref/libftref_server.so not built")
    return RefEngine(threads=2, cpus=sorted(os.sched_getaffinity(0))[:2], path=REFLIB_SERVER)


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import _native
    return _native.Context(0)
