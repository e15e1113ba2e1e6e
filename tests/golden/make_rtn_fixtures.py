"""Writes tests/golden/rtn_fixtures.safetensors: seeded input/output vectors of the reference's round-to-nearest
weight quantisers, ``quantize_w4_rtn`` and ``quantize_w8_rtn`` (forge/kernels/layouts/rtn.py:27-72).

Their exact fp16 / bf16 scale double rounding and ``clamp_min(1e-12)`` order are fixed only by the reference's own
code, so this script imports it -- in the build container only, where the reference tree is mounted (default
/root/reference, or $FORGE_REFERENCE).  The committed file holds data only: inputs and the reference's outputs.
Nothing on the GPU box runs this script; tests read the fixture file.

    python tests/golden/make_rtn_fixtures.py
"""
from __future__ import annotations

import json
import os
import sys

import torch
from safetensors.torch import save_file

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rtn_fixtures.safetensors")

# (n, k, group_size, sym, scale dtype) for W4, (n, k, group_size, scale dtype) for W8
W4_CASES = [(8, 256, 128, True, "float16"), (8, 256, 128, False, "float16"), (8, 200, 64, False, "bfloat16"),
            (8, 200, 64, True, "bfloat16"), (6, 96, -1, False, "float32"), (6, 96, -1, True, "float16"),
            (4, 136, 32, False, "float16")]
W8_CASES = [(8, 256, -1, "float16"), (8, 200, 64, "bfloat16"), (6, 128, 32, "float32")]


def weights(n: int, k: int, seed: int) -> torch.Tensor:
    """N(0, 0.05) rows, then special rows: all zeros, tiny values (the scale underflows fp16 and is re-clamped),
    an outlier, a constant row, and an all-positive row (asymmetric zero-point at 0)."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.05
    w[1] = 0.0
    w[2] = torch.randn(k, generator=g) * 1e-9
    if n > 3:
        w[3, k // 3] = 7.5
    if n > 4:
        w[4] = 0.3125
    if n > 5:
        w[5] = torch.rand(k, generator=g) * 0.1 + 0.01
    return w


def main() -> None:
    ref = os.environ.get("FORGE_REFERENCE", "/root/reference")
    sys.path.insert(0, ref)
    from forge.kernels.layouts.rtn import quantize_w4_rtn, quantize_w8_rtn

    tensors: dict[str, torch.Tensor] = {}
    meta = {"w4": [], "w8": []}
    for i, (n, k, gs, sym, sdt) in enumerate(W4_CASES):
        w = weights(n, k, 100 + i)
        q, s, z = quantize_w4_rtn(w, gs, sym=sym, scale_dtype=getattr(torch, sdt))
        tensors[f"w4_{i}_w"], tensors[f"w4_{i}_q"], tensors[f"w4_{i}_s"] = w, q, s
        if z is not None:
            tensors[f"w4_{i}_z"] = z
        meta["w4"].append({"n": n, "k": k, "group_size": gs, "sym": sym, "scale_dtype": sdt})
    for i, (n, k, gs, sdt) in enumerate(W8_CASES):
        w = weights(n, k, 200 + i)
        q, s = quantize_w8_rtn(w, gs, scale_dtype=getattr(torch, sdt))
        tensors[f"w8_{i}_w"], tensors[f"w8_{i}_q"], tensors[f"w8_{i}_s"] = w, q, s
        meta["w8"].append({"n": n, "k": k, "group_size": gs, "scale_dtype": sdt})
    save_file({k: v.contiguous() for k, v in tensors.items()}, OUT,
              metadata={"cases": json.dumps(meta), "source": "forge/kernels/layouts/rtn.py:27-72"})
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
