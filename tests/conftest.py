"""Test configuration: import paths and the ``gpu`` marker.

``gpu`` tests need a HIP device and the built ``libramnet_hip.so``; they are
skipped (never run on a fallback) when no GPU is visible.
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (REPO, os.path.join(REPO, "ram-net_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device and the built operator library")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def golden():
    """Load a JSON fixture from tests/golden ('-inf' strings become float -inf)."""
    import json

    def load(name):
        with open(os.path.join(REPO, "tests", "golden", name)) as fh:
            data = json.load(fh)
        if "addr" in data:
            data["addr"] = [float("-inf") if v == "-inf" else v for v in data["addr"]]
        return data
    return load
