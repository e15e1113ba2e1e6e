"""The device self-test (known-answer W4A16 / INT8 / FP8 checks run on first use of a device) passes, and a
kernel result that breaks its closed form is reported."""
from __future__ import annotations

import pytest
import torch

from forge_amd import ops_gemm as ops

pytestmark = pytest.mark.gpu


def test_device_selftest_passes():
    assert ops.device_selftest(0) == []


def test_selftest_reports_a_wrong_answer(monkeypatch):
    real = ops.int8_gemm
    monkeypatch.setattr(ops, "int8_gemm", lambda *a, **k: real(*a, **k) + 1)  # a planted off-by-one on the host side
    assert ops.device_selftest(0) == ["int8"]
    assert torch.cuda.is_available()
