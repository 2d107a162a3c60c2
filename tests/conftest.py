"""Shared pytest configuration: the ``gpu`` marker and repository imports."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


def load_golden(name):
    with np.load(os.path.join(GOLDEN, f"golden_{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session", params=["c1", "c2", "c3"])
def golden(request):
    g = load_golden(request.param)
    g["name"] = request.param
    return g
