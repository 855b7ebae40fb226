"""Shared fixtures. GPU tests are marked `gpu`; everything else runs on a CPU-only machine."""
import importlib
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pkg(name: str):
    """A module of the package (its directory name has a hyphen, so it is imported by name)."""
    return importlib.import_module(f"tabicl-anywhere_amd.{name}")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on the card)")


@pytest.fixture(scope="session")
def tiny_model():
    B, M = pkg("bundle"), pkg("model")
    return M.Model.load(B.Bundle.open(os.path.join(GOLDEN, "tiny-clf.tirs")))


@pytest.fixture(scope="session")
def tiny_raw():
    return pkg("bundle").Bundle.open(os.path.join(GOLDEN, "tiny-raw.tirs"))


def to_ours(r, heads, n, hd):
    """Reference keys/values `[heads][n][hd]` to the dimension-major `[d][n]` (tests/reference.rs:27-37)."""
    r = np.asarray(r).reshape(heads, n, hd)
    return np.transpose(r, (0, 2, 1)).reshape(heads * hd, n)
