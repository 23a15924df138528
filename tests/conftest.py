import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "sepal-runner_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")


@pytest.fixture(scope="session")
def golden():
    """The committed fixtures dumped from the reference's own CPU build (tests/golden/make_golden.py)."""
    import numpy as np
    d = os.path.join(ROOT, "tests", "golden")
    return {name: np.load(os.path.join(d, name + ".npz"), allow_pickle=False)
            for name in ("ref_suite", "ref_mlp", "ref_rmsnorm", "ref_i8y")}
