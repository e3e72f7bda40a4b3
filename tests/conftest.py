import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libkfhip.so")


def pytest_collection_modifyitems(config, items):
    import torch

    has_gpu = torch.cuda.is_available() and torch.version.hip is not None
    skip = pytest.mark.skip(reason="no ROCm GPU")
    for item in items:
        if "gpu" in item.keywords and not has_gpu:
            item.add_marker(skip)
