"""Test configuration: import paths, the ``gpu`` marker, and GPU auto-skip when no HIP device is visible."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "forge-llm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu on the GPU box")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch):
    for v in ("FORGE_FORCE_REF", "FORGE_W4_IMPL", "FORGE_KERNEL_DEBUG"):
        monkeypatch.delenv(v, raising=False)
