"""Test configuration: the `gpu` marker, import paths, shared generators."""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "oracle"), os.path.join(REPO, "esp32-needle-3_amd"),
          os.path.join(REPO, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def normal(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


@pytest.fixture
def rng():
    return np.random.default_rng(20261201)
