"""GPU parity of the decode GEMV on 8-channel scale blocks (fg_w4a16_gemv_sz8: the copy of a portable_row weight's
scales / zero words that KernelW4A16Linear.prepare keeps, forge_amd.layouts.sz8_blocks): bit-identical to the split-K
GEMV on the portable_row tensors (fg_w4a16_gemm) on the Llama-3-8B shapes at full size and on smaller shapes with
fp16 x, bf16 scales, bias, symmetric weights and groups of 32 / 64 / one group, at 1..4 rows; against the fp32 oracle
on one case; the module path at 1 and 2 rows; a stale copy (scales changed in place) not used; graph replays;
host-side rejections (N % 8, n_groups) before any launch.

Bar: bit-identical to the portable GEMV (same arithmetic, same order) and max|y - ref| / max|ref| <= 1e-2 of the
oracle (forge/kernels/ref/gemm_w4a16.py:45-52 restated in oracle/gemm.py)."""
from __future__ import annotations

import pytest
import torch

from forge_amd import _lib
from forge_amd import layouts as L
from forge_amd import ops_gemm as ops
from oracle import gemm as og
from tests._util import assert_close, oracle_packed, to_f32, w4_parts, x_act

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _sz8(x, p, s8, z8, bias=None, n_groups=None):
    m, k = x.shape
    y = torch.full((m, p.n), float("nan"), dtype=x.dtype, device=DEV)
    rc = _lib.lib().fg_w4a16_gemv_sz8(
        _lib.ptr(x), x.stride(0), _lib.dtype_code(x.dtype), _lib.ptr(p.qweight), p.qweight.stride(0), _lib.ptr(s8),
        _lib.dtype_code(s8.dtype), _lib.ptr(z8), _lib.ptr(bias), 0 if bias is None else _lib.dtype_code(bias.dtype),
        _lib.ptr(y), y.stride(0), m, p.n, k, p.group_size, p.num_groups if n_groups is None else n_groups,
        _lib.stream_of(x))
    return rc, y


CASES = [  # m, n, k, gs, sym, x dtype, scale dtype, bias
    (1, 6144, 4096, 128, False, torch.bfloat16, torch.float16, False),    # qkv
    (1, 4096, 4096, 128, False, torch.bfloat16, torch.float16, False),    # o_proj
    (1, 28672, 4096, 128, False, torch.bfloat16, torch.float16, False),   # gate+up
    (1, 4096, 14336, 128, False, torch.bfloat16, torch.float16, False),   # down (7 K slices)
    (2, 28672, 4096, 128, False, torch.bfloat16, torch.float16, True),
    (2, 4096, 14336, 128, True, torch.float16, torch.bfloat16, True),
    (3, 1024, 2048, 64, False, torch.float16, torch.float16, False),
    (4, 520, 1024, 32, False, torch.bfloat16, torch.bfloat16, True),
    (1, 2048, 3072, -1, False, torch.bfloat16, torch.float16, False),     # one group per row
    (1, 8192, 28672, 128, False, torch.bfloat16, torch.float16, False),   # 16 rows per wavefront
]


@pytest.mark.parametrize("m,n,k,gs,sym,xdt,sdt,has_bias", CASES)
def test_sz8_gemv_is_bit_identical_to_the_portable_gemv(m, n, k, gs, sym, xdt, sdt, has_bias):
    q, s, z = w4_parts(n, k, gs, sym, seed=m + n + k, scale_dtype=sdt)
    p = L.pack_w4(q, s, z, gs).to(DEV)
    x = x_act(m, k, xdt, seed=m + 3).to(DEV)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.5).to(xdt).to(DEV) if has_bias else None
    s8, z8 = L.sz8_blocks(p.scales, p.zeros, n)
    rc, y = _sz8(x, p, s8, z8, bias)
    assert rc == _lib.OK, _lib.last_error()
    kern = _lib.last_kernel()
    assert "w4_gemv_split_kernel" in kern and "sz8" in kern, kern
    ref = ops.w4a16_linear(x, p, bias, config={"impl": "gemv"})
    assert "w4_gemv_split_kernel" in ops.last_kernel() and "sz8" not in ops.last_kernel(), ops.last_kernel()
    assert torch.equal(y, ref), f"m={m} n={n} k={k}: not bit-identical to the portable GEMV"


def test_sz8_gemv_matches_the_oracle():
    m, n, k, gs = 2, 1536, 4096, 128
    q, s, z = w4_parts(n, k, gs, False, seed=7)
    p = L.pack_w4(q, s, z, gs).to(DEV)
    x = x_act(m, k, torch.bfloat16, seed=8).to(DEV)
    rc, y = _sz8(x, p, *L.sz8_blocks(p.scales, p.zeros, n))
    assert rc == _lib.OK, _lib.last_error()
    assert_close(y.cpu(), og.w4a16_gemm_ref(to_f32(x.cpu()), oracle_packed(q, s, z, gs)), "bfloat16", what="sz8")


@pytest.mark.parametrize("m", [1, 2, 3])
def test_module_serves_one_and_two_rows_from_the_blocks(m):
    """KernelW4A16Linear keeps the blocks beside the portable tensors (state dict unchanged) and its 1..2-row calls
    run the sz8 GEMV, bit-identical to the portable GEMV; 3 rows go to the CDNA4-layout copy."""
    n, k, gs = 4096, 4096, 128
    q, s, z = w4_parts(n, k, gs, False, seed=m + 60)
    packed = L.pack_w4(q, s, z, gs).to(DEV)
    mod = ops.KernelW4A16Linear.from_packed(packed)
    x = x_act(m, k, torch.bfloat16, seed=m + 61).to(DEV)
    y = mod(x)
    kern = ops.last_kernel()
    assert ("sz8" in kern) == (m <= ops.SZ8_ROWS), kern
    if m <= ops.SZ8_ROWS:
        assert torch.equal(y, ops.w4a16_linear(x, packed, config={"impl": "gemv"}))
    assert not any("sz8" in key for key in mod.state_dict()) and mod.state_dict()["scales"].shape == packed.scales.shape
    assert_close(y.cpu(), og.w4a16_gemm_ref(to_f32(x.cpu()), oracle_packed(q, s, z, gs)), "bfloat16",
                 what=f"module m={m}")


def test_stale_blocks_are_not_used():
    """Scales changed in place after the blocks were made: the op notices (tensor version) and reads the portable
    tensors, so the result follows the new scales."""
    n, k, gs = 2048, 2048, 128
    q, s, z = w4_parts(n, k, gs, False, seed=70)
    p = L.pack_w4(q, s, z, gs).to(DEV)
    assert ops.prepare_w4_sz8(p)
    x = x_act(1, k, torch.bfloat16, seed=71).to(DEV)
    ops.w4a16_linear(x, p)
    assert "sz8" in ops.last_kernel()
    p.scales.mul_(2)
    y = ops.w4a16_linear(x, p)
    assert "sz8" not in ops.last_kernel()
    assert torch.equal(y, ops.w4a16_linear(x, p, config={"impl": "gemv"}))


def test_sz8_gemv_in_a_graph_replays_like_eager():
    n, k, gs = 6144, 4096, 128
    q, s, z = w4_parts(n, k, gs, False, seed=80)
    p = L.pack_w4(q, s, z, gs).to(DEV)
    assert ops.prepare_w4_sz8(p)
    x = x_act(1, k, torch.bfloat16, seed=81).to(DEV)
    eager = ops.w4a16_linear(x, p).clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ops.w4a16_linear(x, p)
    torch.cuda.current_stream().wait_stream(st)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ops.w4a16_linear(x, p)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_sz8_rejections_happen_before_any_launch():
    n, k, gs = 1024, 1024, 128
    q, s, z = w4_parts(n, k, gs, False, seed=90)
    p = L.pack_w4(q, s, z, gs).to(DEV)
    x = x_act(1, k, torch.bfloat16, seed=91).to(DEV)
    s8, z8 = L.sz8_blocks(p.scales, p.zeros, n)
    rc, _ = _sz8(x, p, s8, z8, n_groups=p.num_groups + 1)
    assert rc == _lib.EINVAL and "n_groups" in _lib.last_error()
    rc, _ = _sz8(x_act(5, k, torch.bfloat16, seed=92).to(DEV), p, s8, z8)
    assert rc == _lib.EUNSUPPORTED
    odd = L.pack_w4(*w4_parts(1020, k, gs, False, seed=93), gs).to(DEV)
    rc, _ = _sz8(x, odd, s8, z8)
    assert rc == _lib.EUNSUPPORTED and "N % 8" in _lib.last_error()
