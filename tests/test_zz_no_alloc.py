"""fg_w4a16_gemm_noalloc (split-K partials in the library's static scratch buffer, no allocation) against
fg_w4a16_gemm with a caller workspace, through the C ABI: two calls in a row, the second on a smaller problem, each
bit-identical to the workspace entry point on the same operands (the same kernels run); a plan that needs more
scratch than the buffer holds is rejected before any launch."""
from __future__ import annotations

import ctypes

import pytest
import torch

from forge_amd import _lib
from forge_amd import layouts as L
from tests._util import w4_parts, x_act

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _args(x, p, y, cfg):
    m, k = x.shape
    return [_lib.ptr(x), x.stride(0), _lib.dtype_code(x.dtype), _lib.ptr(p.qweight), p.qweight.stride(0),
            _lib.ptr(p.scales), _lib.dtype_code(p.scales.dtype), p.scales.stride(0), _lib.ptr(p.zeros),
            0 if p.zeros is None else p.zeros.stride(0), None, None, None, 0, _lib.ptr(y), y.stride(0), m, p.n, k,
            p.group_size, p.num_groups, None if cfg is None else ctypes.byref(cfg)]


def _both(m, n, k, seed, cfg=None):
    q, s, z = w4_parts(n, k, 128, False, seed=seed)
    p = L.pack_w4(q, s, z, 128).to(DEV)
    x = x_act(m, k, torch.bfloat16, seed=seed + 1).to(DEV)
    lib = _lib.lib()
    stream = _lib.stream_of(x)
    ws_bytes = lib.fg_w4a16_workspace_bytes(m, n, k, 128, 1, 1, 0, None if cfg is None else ctypes.byref(cfg))
    assert 0 < ws_bytes <= _lib.W4A16_SCRATCH_BYTES
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    y_ws = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    y_na = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.fg_w4a16_gemm(*_args(x, p, y_ws, cfg), _lib.ptr(ws), ws_bytes, stream), "fg_w4a16_gemm")
    kern_ws = _lib.last_kernel()
    _lib.check(lib.fg_w4a16_gemm_noalloc(*_args(x, p, y_na, cfg), stream), "fg_w4a16_gemm_noalloc")
    assert _lib.last_kernel() == kern_ws, "both entry points must run the same kernels"
    torch.cuda.synchronize()
    return y_ws, y_na, kern_ws


def test_noalloc_matches_workspace_entry_point_twice():
    # 64 rows over down (K = 14336): the LDS-ring kernel with 8 K splits, whose 8.4 MB of fp32 partials go to the
    # scratch buffer and are summed by its reduce kernel
    y_ws, y_na, kern = _both(64, 4096, 14336, seed=1)
    assert "w4_ring_kernel" in kern and "KS=8" in kern and "reduce" in kern, kern
    assert torch.equal(y_ws, y_na)
    # then a smaller problem (40 rows over qkv: the ring kernel with 4 K splits, 3.9 MB): the first call's partials
    # stay behind it in the buffer
    y_ws, y_na, kern = _both(40, 6144, 4096, seed=2)
    assert "w4_ring_kernel" in kern and "reduce" in kern, kern
    assert torch.equal(y_ws, y_na)
    # and a forced split count through the tiled MFMA kernel's split-K path
    cfg = _lib.W4Config(_lib.W4_MFMA, 0, 0, 32, 4)
    y_ws, y_na, kern = _both(24, 2048, 4096, seed=3, cfg=cfg)
    assert "w4_mfma_kernel splits=4" in kern, kern
    assert torch.equal(y_ws, y_na)


def test_noalloc_rejects_plans_beyond_the_scratch_buffer():
    m, n, k = 1000, 4096, 4096
    cfg = _lib.W4Config(_lib.W4_PREFILL, 0, 0, 0, 8)  # 8 K splits of 1000 x 4096 fp32 partials: 131 MB
    lib = _lib.lib()
    assert lib.fg_w4a16_workspace_bytes(m, n, k, 128, 1, 1, 0, ctypes.byref(cfg)) > _lib.W4A16_SCRATCH_BYTES
    q, s, z = w4_parts(n, k, 128, False, seed=4)
    p = L.pack_w4(q, s, z, 128).to(DEV)
    x = x_act(m, k, torch.bfloat16, seed=5).to(DEV)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    rc = lib.fg_w4a16_gemm_noalloc(*_args(x, p, y, cfg), _lib.stream_of(x))
    assert rc == _lib.EINVAL and "static buffer" in _lib.last_error()
