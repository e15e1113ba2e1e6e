"""Shared helpers: seeded synthetic inputs in the distributions of BASELINE.json's configs, torch <-> oracle bridges."""
from __future__ import annotations

import numpy as np
import torch

from forge_amd import layouts
from oracle import gemm as og
from oracle import w4 as ow


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def w4_parts(n: int, k: int, gs: int, sym: bool, seed: int = 0, scale_dtype=torch.float16):
    """q ~ U{0..15}, scales ~ U[0.002, 0.02] (rounded to scale_dtype), zeros ~ U{6..9} (None when symmetric)."""
    g = gen(seed)
    ng = layouts.num_groups(k, gs)
    q = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8)
    s = (torch.rand(n, ng, generator=g) * 0.018 + 0.002).to(scale_dtype)
    z = None if sym else torch.randint(6, 10, (n, ng), generator=g, dtype=torch.uint8)
    return q, s, z


def oracle_packed(q, s, z, gs, g_idx=None) -> dict:
    """Oracle packing of the same logical parts (scales widened to float32 exactly)."""
    return ow.pack_w4(q.numpy(), s.float().numpy(), None if z is None else z.numpy(), gs,
                      None if g_idx is None else g_idx.numpy())


def x_act(m: int, k: int, dtype=torch.bfloat16, seed: int = 1, scale: float = 1.0) -> torch.Tensor:
    return (torch.randn(m, k, generator=gen(seed)) * scale).to(dtype)


def to_f32(t: torch.Tensor) -> np.ndarray:
    """Exact widening of a bf16/fp16/fp32 CPU tensor to a float32 numpy array."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return og.bf16_to_f32(t.view(torch.int16).numpy().view(np.uint16))
    return t.float().numpy()


def fp8_codes(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.uint8).numpy()


def assert_close(out: torch.Tensor, ref: np.ndarray, out_dtype: str, *, rel: float = 1e-2, what: str = ""):
    """North-star bar (max |out - ref| / max |ref| <= 1e-2) and the reference's compare() spec rule."""
    o = to_f32(out)
    r = og.max_rel_err(o, ref)
    assert r <= rel, f"{what}: max rel err {r:.3e} > {rel}"
    res = og.compare(o, ref, out_dtype=out_dtype)
    assert res["ok"], f"{what}: {res['detail']}"
    return r
