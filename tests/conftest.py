"""pytest setup: repo root and oracle/ on sys.path, the `gpu` marker, shared fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm GPU) and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    if not os.path.isfile(o.LIB_PATH):
        o.build_lib()
    return o


@pytest.fixture(scope="session")
def hip():
    """The product package with its HIP backend loaded; fails (not skips) when the library cannot run on a GPU box."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this process")
    import lfm3_kv800_amd.kv800_hip as kh
    kh.ops()
    return kh
