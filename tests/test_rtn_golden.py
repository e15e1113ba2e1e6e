"""The RTN weight quantisers (load-time producers behind ``from_dense``) against vectors the reference's own
``quantize_w4_rtn`` / ``quantize_w8_rtn`` wrote (forge/kernels/layouts/rtn.py:27-72; tests/golden/make_rtn_fixtures.py
generated them in the build container).  Codes, scales (dtype and bits) and zero-points must be equal."""
from __future__ import annotations

import json
import os

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import load_file

from forge_amd import layouts as L

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rtn_fixtures.safetensors")
T = load_file(FIX)
with safe_open(FIX, "pt") as f:
    CASES = json.loads(f.metadata()["cases"])


@pytest.mark.parametrize("i", range(len(CASES["w4"])))
def test_quantize_w4_rtn_matches_reference_vectors(i):
    c = CASES["w4"][i]
    q, s, z = L.quantize_w4_rtn(T[f"w4_{i}_w"], c["group_size"], sym=c["sym"], scale_dtype=getattr(torch, c["scale_dtype"]))
    assert q.dtype == torch.uint8 and torch.equal(q, T[f"w4_{i}_q"])
    assert s.dtype == T[f"w4_{i}_s"].dtype and torch.equal(s.view(torch.uint8), T[f"w4_{i}_s"].view(torch.uint8))
    if c["sym"]:
        assert z is None and f"w4_{i}_z" not in T
    else:
        assert torch.equal(z, T[f"w4_{i}_z"])


@pytest.mark.parametrize("i", range(len(CASES["w8"])))
def test_quantize_w8_rtn_matches_reference_vectors(i):
    c = CASES["w8"][i]
    q, s = L.quantize_w8_rtn(T[f"w8_{i}_w"], c["group_size"], scale_dtype=getattr(torch, c["scale_dtype"]))
    assert q.dtype == torch.int8 and torch.equal(q, T[f"w8_{i}_q"])
    assert s.dtype == T[f"w8_{i}_s"].dtype and torch.equal(s.view(torch.uint8), T[f"w8_{i}_s"].view(torch.uint8))


def test_fixture_cases_cover_the_edge_rows():
    """Zero rows (scale clamped to 1e-12 twice), underflowing fp16 scales, outliers, K not a multiple of the group."""
    w = T["w4_0_w"]
    assert (w[1] == 0).all() and w[2].abs().max() < 1e-8 and w[3].abs().max() == 7.5
    assert any(c["k"] % c["group_size"] for c in CASES["w4"] if c["group_size"] > 0)
    assert {c["scale_dtype"] for c in CASES["w4"]} == {"float16", "bfloat16", "float32"}
