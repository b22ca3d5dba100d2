"""Test configuration: markers, repo on sys.path, thread count.

Markers: ``gpu`` (needs an MI355X and the built HIP library; run with
``-m gpu``), everything else runs on the CPU.  As the reference's own
conftest.py:13 does, CPU math runs single-threaded so results do not depend
on the host's core count.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
os.environ.setdefault("OMP_NUM_THREADS", "1")

import pytest  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires an AMD GPU (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from wanferenz_amd import _native

    _native.lib()
    return torch.device("cuda:0")
