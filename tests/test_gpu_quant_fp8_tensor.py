"""FP8 quantisation with few, large scale tiles (per tensor; 1024 x 1024 blocks): the tile is cut into parts
reduced by many workgroups (atomic max of the amax bit patterns in the scale buffer), or, for a static per-tensor
scale, quantised row by row.  Codes and scales bit-exact against the oracle (forge/kernels/ref/gemm_fp8.py:43-85),
NaN and all-zero inputs included."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from forge_amd import _lib
from forge_amd import ops_gemm as ops
from oracle import gemm as og
from tests._util import fp8_codes, gen, to_f32

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("m,k", [(4096, 8192), (3, 70000), (1, 100)])
def test_per_tensor_dynamic_matches_oracle(m, k):
    x = (torch.randn(m, k, generator=gen(m + k)) * 2).to(torch.bfloat16)
    x[m // 2, k // 3] = 37.5  # the amax sits in one part
    q, s = ops.quantize_act_fp8(x.to(DEV), granularity="per_tensor")
    qr, sr = og.quantize_fp8_ref(to_f32(x), "per_tensor")
    assert np.array_equal(s.cpu().numpy(), sr) and np.array_equal(fp8_codes(q), qr)


def test_per_tensor_dynamic_nan_and_zeros():
    x = torch.zeros(512, 4096, dtype=torch.bfloat16)
    q, s = ops.quantize_act_fp8(x.to(DEV), granularity="per_tensor")
    assert s.item() == 1.0 and fp8_codes(q).max() == 0
    x = torch.randn(512, 4096, generator=gen(3)).to(torch.bfloat16)
    x[100, 7] = float("nan")
    q, s = ops.quantize_act_fp8(x.to(DEV), granularity="per_tensor")
    qr, sr = og.quantize_fp8_ref(to_f32(x), "per_tensor")
    assert np.array_equal(s.cpu().numpy(), sr) and np.array_equal(fp8_codes(q), qr)


def test_per_tensor_static_rowwise():
    x = (torch.randn(4096, 8192, generator=gen(9)) * 4).to(torch.bfloat16)
    st = torch.tensor([0.0125])
    q, s = ops.quantize_act_fp8(x.to(DEV), granularity="per_tensor", scale=st.to(DEV))
    qr, sr = og.quantize_fp8_ref(to_f32(x), "per_tensor", scale=st.numpy())
    assert np.array_equal(s.cpu().numpy(), sr) and np.array_equal(fp8_codes(q), qr)


def _block_quant(x: torch.Tensor, bm: int, bk: int, static: torch.Tensor | None):
    m, k = x.shape
    q = torch.empty(m, k, dtype=torch.uint8, device=DEV)
    s = None if static is not None else torch.empty(-(-m // bm), -(-k // bk), dtype=torch.float32, device=DEV)
    _lib.check(_lib.lib().fg_quant_fp8_block(_lib.ptr(x), x.stride(0), _lib.dtype_code(x.dtype), _lib.ptr(q), k,
                                             _lib.ptr(s), -(-k // bk), m, k, bm, bk, _lib.ptr(static),
                                             _lib.stream_of(x)), "fg_quant_fp8_block")
    return q, s


def test_c_abi_large_blocks_dynamic_and_static():
    """2 x 4 blocks of 1024 x 1024 (ragged last column block): dynamic scales per block, and one static scale for
    all blocks (every part must read the same value)."""
    x = (torch.randn(2048, 3900, generator=gen(11)) * 3).to(torch.bfloat16)
    x[1500, 3100] = -90.0
    q, s = _block_quant(x.to(DEV), 1024, 1024, None)
    qr, sr = og.quantize_fp8_ref(to_f32(x), "block2d", block=1024)
    assert np.array_equal(s.cpu().numpy(), sr) and np.array_equal(q.cpu().numpy(), qr)
    st = torch.tensor([0.02], device=DEV)
    q2, _ = _block_quant(x.to(DEV), 1024, 1024, st)
    qr2, _ = og.quantize_fp8_ref(to_f32(x), "per_tensor", scale=np.array([0.02], np.float32))
    assert np.array_equal(q2.cpu().numpy(), qr2)
