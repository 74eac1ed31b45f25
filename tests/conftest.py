import importlib
import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")
    config.addinivalue_line("markers", "slow: full-size configurations")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def pkg():
    return importlib.import_module("artifex-assistantv5_amd")


@pytest.fixture(scope="session")
def ref():
    from oracle import gguf_ref
    return gguf_ref


@pytest.fixture(scope="session")
def golden_samples():
    with open(os.path.join(GOLDEN, "gguf_dequant_samples.json"), encoding="utf-8") as f:
        return json.load(f)["samples"]


@pytest.fixture(scope="session")
def synthetic_small():
    return dict(np.load(os.path.join(GOLDEN, "synthetic_small.npz")))
