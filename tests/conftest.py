"""pytest configuration: the ``gpu`` marker and import paths.

``-m "not gpu"`` runs on any host (oracle pins, API/dispatch logic, C-ABI
load and argument checks); ``-m gpu`` runs the HIP kernels against the oracle
and needs an MI355X.
"""
import os
import sys

import pytest

# A module asked for its kernel path with the extension missing raises instead
# of running its PyTorch path: a test must never pass on the fallback.
os.environ.setdefault("GENIE_TK_STRICT", "1")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "genie-tk_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU and the built HIP extension")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
