"""GPU parity of the skinny W8A8 kernel (fg_w8_skinny.hip, M <= 64, register-resident split-K): INT8 accumulator and
fp32 / bf16 / fp16 epilogues bit-exact against the CPU oracle (the int32 partials of the K slices sum exactly), FP8
within the north-star bar, as is the 64-row kernel on the same inputs; forced with tile_m=16, and the policy's own choice
(the skinny kernel for M <= 16 at K >= 16384 and for M <= 32 where the ring's 64 x 32 tiles would not cover the CUs,
the ring kernel for the other aligned shapes) held to the same bar."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from forge_amd import _lib
from forge_amd import ops_gemm as ops
from oracle import gemm as og
from tests._util import assert_close, gen, to_f32

pytestmark = pytest.mark.gpu
DEV = "cuda"
SK = {"tile_m": 16}


def _i8(m, n, k, seed):
    x = torch.randn(m, k, generator=gen(seed)).numpy()
    w = (torch.randn(n, k, generator=gen(seed + 1)) * 0.05).numpy()
    xq, sx = og.quantize_int8_ref(x, "per_token")
    wq, sw = og.quantize_int8_ref(w, "per_channel")
    return xq, sx, wq, sw


@pytest.mark.parametrize("m,n,k", [(1, 10240, 8192), (5, 777, 256), (16, 4096, 2048), (17, 1000, 512),
                                   (33, 520, 1024), (64, 2048, 4096), (3, 96, 28672)])
def test_skinny_int8_exact_vs_oracle(m, n, k):
    xq, sx, wq, sw = _i8(m, n, k, seed=m + n + k)
    a, w = torch.from_numpy(xq).to(DEV), torch.from_numpy(wq).to(DEV)
    acc = ops.int8_gemm(a, None, w, None, out_dtype=torch.int32, config=SK).cpu().numpy()
    ref_acc = og.int8_matmul_exact(xq, wq)
    assert np.array_equal(acc, ref_acc)
    b = torch.randn(n, generator=gen(9))
    ta, tb = torch.from_numpy(sx).to(DEV), torch.from_numpy(sw).to(DEV)
    y32 = ops.int8_gemm(a, ta, w, tb, b.to(DEV), out_dtype=torch.float32, config=SK).cpu().numpy()
    ref32 = og.int8_gemm_ref(xq, sx, wq, sw, b.numpy(), acc=ref_acc)
    assert np.array_equal(y32, ref32)
    for odt in (torch.bfloat16, torch.float16):
        y16 = ops.int8_gemm(a, ta, w, tb, b.to(DEV), out_dtype=odt).cpu()  # the policy's kernel
        assert torch.equal(y16, torch.from_numpy(ref32).to(odt)), odt


@pytest.mark.parametrize("m,n,k", [(1, 8192, 8192), (16, 8192, 8192), (7, 1000, 512), (40, 256, 1024),
                                   (64, 4096, 2048)])
def test_skinny_fp8_vs_oracle_and_tiled(m, n, k):
    x = torch.randn(m, k, generator=gen(m + k)).to(torch.bfloat16)
    w = torch.randn(n, k, generator=gen(n)) * 0.05
    xq, sx = og.quantize_fp8_ref(to_f32(x), "per_token")
    wq, sw = og.quantize_fp8_ref(w.numpy(), "per_channel")
    txq = torch.from_numpy(xq).view(torch.float8_e4m3fn).to(DEV)
    twq = torch.from_numpy(wq).view(torch.float8_e4m3fn).to(DEV)
    tsx, tsw = torch.from_numpy(sx).to(DEV), torch.from_numpy(sw).to(DEV)
    b = (torch.randn(n, generator=gen(4)) * 0.1).to(torch.bfloat16).to(DEV)
    ref = og.fp8_gemm_ref(xq, sx, wq, sw, to_f32(b.cpu()))
    for odt in (torch.bfloat16, torch.float16, torch.float32):
        y = ops.fp8_linear(txq, twq, tsw, b, x_scale=tsx, out_dtype=odt, config=SK)
        y64 = ops.fp8_linear(txq, twq, tsw, b, x_scale=tsx, out_dtype=odt, config={"tile_m": 64})
        name = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}[odt]
        assert_close(y.cpu(), ref, name, what=f"fp8 skinny m={m} {name}")
        assert_close(y64.cpu(), ref, name, what=f"fp8 tiled m={m} {name}")
    # per-tensor scales (mode 0) through the same kernel
    s1 = torch.tensor([0.02], device=DEV)
    y0 = ops.fp8_linear(txq, twq, s1, x_scale=s1, out_dtype=torch.float32, config=SK)
    ref0 = og.fp8_gemm_ref(xq, np.float32([0.02]), wq, np.float32([0.02]))
    assert_close(y0.cpu(), ref0, "float32", what="fp8 skinny per-tensor")


def test_skinny_reproducible_and_rejects():
    g = torch.Generator(device=DEV).manual_seed(3)
    a = torch.randint(-127, 128, (24, 8192), dtype=torch.int8, device=DEV, generator=g)
    w = torch.randint(-127, 128, (4096, 8192), dtype=torch.int8, device=DEV, generator=g)
    runs = [ops.int8_gemm(a, None, w, None, out_dtype=torch.int32) for _ in range(3)]
    assert all(torch.equal(runs[0], r) for r in runs[1:])
    a2 = torch.zeros(8, 1000, dtype=torch.int8, device=DEV)
    w2 = torch.zeros(64, 1000, dtype=torch.int8, device=DEV)
    with pytest.raises(_lib.KernelLaunchError, match="tile_m=16"):
        ops.int8_gemm(a2, None, w2, None, out_dtype=torch.int32, config=SK)  # K % 256 != 0
    assert ops.int8_gemm(a2, None, w2, None, out_dtype=torch.int32).abs().sum().item() == 0  # policy falls back


@pytest.mark.parametrize("m,n,k", [(4, 4096, 14336), (24, 4096, 14336), (8, 4096, 4096), (32, 2048, 4096)])
def test_policy_skinny_for_narrow_outputs(m, n, k):
    """M <= 32 over N < 32 x CUs (fewer 64 x 32 ring tiles than CUs): the policy's INT8 and FP8 results equal the forced
    skinny kernel's bit for bit and match the oracle (INT8 bf16 output exactly)."""
    xq, sx, wq, sw = _i8(m, n, k, seed=m + n + k)
    a, w = torch.from_numpy(xq).to(DEV), torch.from_numpy(wq).to(DEV)
    ta, tb = torch.from_numpy(sx).to(DEV), torch.from_numpy(sw).to(DEV)
    y = ops.int8_gemm(a, ta, w, tb, out_dtype=torch.bfloat16)
    assert torch.equal(y, ops.int8_gemm(a, ta, w, tb, out_dtype=torch.bfloat16, config=SK))
    ref = og.int8_gemm_ref(xq, sx, wq, sw, None, acc=og.int8_matmul_exact(xq, wq))
    assert torch.equal(y.cpu(), torch.from_numpy(ref).to(torch.bfloat16))
    x = torch.randn(m, k, generator=gen(m + 7)).to(torch.bfloat16)
    wf = torch.randn(n, k, generator=gen(n + 8)) * 0.05
    fq, fsx = og.quantize_fp8_ref(to_f32(x), "per_token")
    gq, gsw = og.quantize_fp8_ref(wf.numpy(), "per_channel")
    txq = torch.from_numpy(fq).view(torch.float8_e4m3fn).to(DEV)
    twq = torch.from_numpy(gq).view(torch.float8_e4m3fn).to(DEV)
    tsx, tsw = torch.from_numpy(fsx).to(DEV), torch.from_numpy(gsw).to(DEV)
    yf = ops.fp8_linear(txq, twq, tsw, x_scale=tsx, out_dtype=torch.bfloat16)
    assert torch.equal(yf, ops.fp8_linear(txq, twq, tsw, x_scale=tsx, out_dtype=torch.bfloat16, config=SK))
    assert_close(yf.cpu(), og.fp8_gemm_ref(fq, fsx, gq, gsw), "bfloat16", what=f"fp8 policy skinny m={m} n={n} k={k}")
