import json
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GOLDEN = os.path.join(HERE, "golden", "data")
if HERE not in sys.path:
    sys.path.insert(0, HERE)
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")
    config.addinivalue_line("markers", "slow: long CPU-side check, skipped unless QL_SLOW=1")


def pytest_collection_modifyitems(config, items):
    if os.environ.get("QL_SLOW") == "1":
        return
    skip = pytest.mark.skip(reason="slow check; set QL_SLOW=1")
    for it in items:
        if "slow" in it.keywords:
            it.add_marker(skip)


def golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npy"), allow_pickle=False)


def golden_json(name):
    with open(os.path.join(GOLDEN, name + ".json")) as f:
        return json.load(f)


def have_golden(name):
    return os.path.exists(os.path.join(GOLDEN, name))
