"""GPU parity of the small-M W8A8 ring kernel (fg_mm_big.hip mm_ring_kernel: 64- or 128-row tiles, direct-to-LDS
loads through a several-stage LDS ring).  Each instance is forced with tile_m / tile_n on ragged shapes, K from one
128-byte slice to more slices than the ring has stages: INT8 accumulator and fp32 / bf16 / fp16 epilogues bit-exact
against the CPU oracle, FP8 within the north-star bar and bit-identical across instances (same MFMA instruction and K
order).  At the configs' small-M sizes the policy's own choice equals a forced instance and matches the oracle on
sampled rows."""
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
RINGS = [{"tile_m": 64, "tile_n": 32}, {"tile_m": 64, "tile_n": 64}, {"tile_m": 64, "tile_n": 128},
         {"tile_m": 128, "tile_n": 128}]
SHAPES = [(1, 1000, 1024), (37, 517, 128), (100, 300, 384), (200, 1030, 1152), (64, 256, 2048)]


def _i8(m, n, k, seed):
    x = torch.randn(m, k, generator=gen(seed)).numpy()
    w = (torch.randn(n, k, generator=gen(seed + 1)) * 0.05).numpy()
    xq, sx = og.quantize_int8_ref(x, "per_token")
    wq, sw = og.quantize_int8_ref(w, "per_channel")
    return xq, sx, wq, sw


@pytest.mark.parametrize("cfg", RINGS, ids=lambda c: f"{c['tile_m']}x{c['tile_n']}")
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_ring_int8_exact_vs_oracle(m, n, k, cfg):
    xq, sx, wq, sw = _i8(m, n, k, seed=m + n + k)
    a, w = torch.from_numpy(xq).to(DEV), torch.from_numpy(wq).to(DEV)
    acc = ops.int8_gemm(a, None, w, None, out_dtype=torch.int32, config=cfg).cpu().numpy()
    ref_acc = og.int8_matmul_exact(xq, wq)
    assert np.array_equal(acc, ref_acc)
    b = torch.randn(n, generator=gen(9))
    ta, tb = torch.from_numpy(sx).to(DEV), torch.from_numpy(sw).to(DEV)
    y32 = ops.int8_gemm(a, ta, w, tb, b.to(DEV), out_dtype=torch.float32, config=cfg).cpu().numpy()
    ref32 = og.int8_gemm_ref(xq, sx, wq, sw, b.numpy(), acc=ref_acc)
    assert np.array_equal(y32, ref32)
    for odt in (torch.bfloat16, torch.float16):  # 16-bit epilogue (LDS slab, 16-byte or ragged stores)
        y16 = ops.int8_gemm(a, ta, w, tb, b.to(DEV), out_dtype=odt, config=cfg).cpu()
        assert torch.equal(y16, torch.from_numpy(ref32).to(odt)), odt


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_ring_fp8_vs_oracle_all_instances_equal(m, n, k):
    x = torch.randn(m, k, generator=gen(m + 1)).to(torch.bfloat16)
    w = torch.randn(n, k, generator=gen(n + 2)) * 0.05
    xq, sx = og.quantize_fp8_ref(to_f32(x), "per_token")
    wq, sw = og.quantize_fp8_ref(w.numpy(), "per_channel")
    txq = torch.from_numpy(xq).view(torch.float8_e4m3fn).to(DEV)
    twq = torch.from_numpy(wq).view(torch.float8_e4m3fn).to(DEV)
    tsx, tsw = torch.from_numpy(sx).to(DEV), torch.from_numpy(sw).to(DEV)
    b = (torch.randn(n, generator=gen(4)) * 0.1).to(torch.bfloat16).to(DEV)
    ref = og.fp8_gemm_ref(xq, sx, wq, sw, to_f32(b.cpu()))
    for odt, name in ((torch.bfloat16, "bfloat16"), (torch.float16, "float16"), (torch.float32, "float32")):
        ys = [ops.fp8_linear(txq, twq, tsw, b, x_scale=tsx, out_dtype=odt, config=c) for c in RINGS]
        for c, y in zip(RINGS[1:], ys[1:]):
            assert torch.equal(y, ys[0]), (c, name)
        assert_close(ys[0].cpu(), ref, name, what=f"fp8 ring m={m} {name}")
    # per-tensor scales (mode 0) through the same kernel
    s1 = torch.tensor([0.02], device=DEV)
    y0 = ops.fp8_linear(txq, twq, s1, x_scale=s1, out_dtype=torch.float32, config=RINGS[1])
    ref0 = og.fp8_gemm_ref(xq, np.float32([0.02]), wq, np.float32([0.02]))
    assert_close(y0.cpu(), ref0, "float32", what="fp8 ring per-tensor")


@pytest.mark.parametrize("cfg", RINGS, ids=lambda c: f"{c['tile_m']}x{c['tile_n']}")
def test_ring_int8_row_strided_x(cfg):
    """x as a view into wider rows (lda = K + 128): rows are addressed through lda, not K."""
    m, n, k = 70, 300, 640
    xq, sx, wq, sw = _i8(m, n, k, seed=5)
    wide = torch.full((m, k + 128), 99, dtype=torch.int8)
    wide[:, :k] = torch.from_numpy(xq)
    a = wide.to(DEV)[:, :k]
    assert a.stride(0) == k + 128
    w = torch.from_numpy(wq).to(DEV)
    acc = ops.int8_gemm(a, None, w, None, out_dtype=torch.int32, config=cfg).cpu().numpy()
    assert np.array_equal(acc, og.int8_matmul_exact(xq, wq))


def test_ring_config_rejects():
    a = torch.zeros(8, 1000, dtype=torch.int8, device=DEV)
    w = torch.zeros(64, 1000, dtype=torch.int8, device=DEV)
    with pytest.raises(_lib.KernelLaunchError, match="tile_n"):  # K % 128 != 0: no ring kernel for tile_n to pick
        ops.int8_gemm(a, None, w, None, out_dtype=torch.int32, config={"tile_m": 64, "tile_n": 64})
    a = torch.zeros(8, 1024, dtype=torch.int8, device=DEV)
    w = torch.zeros(64, 1024, dtype=torch.int8, device=DEV)
    for bad in ({"tile_m": 64, "tile_n": 96}, {"tile_m": 128, "tile_n": 64}):
        with pytest.raises(_lib.KernelLaunchError, match="tile_n"):
            ops.int8_gemm(a, None, w, None, out_dtype=torch.int32, config=bad)
    # tile_m = 64 without tile_n on such K still runs (square register-staged tiles)
    a = torch.ones(8, 1000, dtype=torch.int8, device=DEV)
    w = torch.ones(64, 1000, dtype=torch.int8, device=DEV)
    assert (ops.int8_gemm(a, None, w, None, out_dtype=torch.int32, config={"tile_m": 64}) == 1000).all()


@pytest.mark.parametrize("m,k,n", [(1, 8192, 10240), (64, 8192, 10240), (64, 28672, 8192), (64, 8192, 57344)])
def test_ring_int8_config_sizes_policy(m, k, n):
    """configs[4] at small M: the policy's kernel (the INT8 decode GEMV at M = 1, the ring kernel's 64-row tiles at
    M = 64, and at M = 64 over N = 57344 the 256-row kernel, whose 224 tiles reach 5/8 of the CUs) equals the forced
    64 x 64 ring instance bit for bit and the oracle on sampled rows (bf16 output, per-token x per-channel scales,
    bias)."""
    g = torch.Generator(device=DEV).manual_seed(m + k + n)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=DEV, generator=g)
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=DEV, generator=g)
    sa = torch.rand(m, device=DEV, generator=g) * 0.01 + 0.001
    sw = torch.rand(n, device=DEV, generator=g) * 0.01 + 0.001
    b = torch.randn(n, device=DEV, generator=g)
    y = ops.int8_gemm(a, sa, w, sw, b, out_dtype=torch.bfloat16)
    kern = ops.last_kernel()
    expect = "int8_gemv_kernel" if m == 1 else ("mm_big_kernel" if n == 57344 else "mm_ring_kernel 64x")
    assert kern.startswith(expect), kern
    y64 = ops.int8_gemm(a, sa, w, sw, b, out_dtype=torch.bfloat16, config={"tile_m": 64, "tile_n": 64})
    assert torch.equal(y, y64)
    rows = sorted({0, m // 2, m - 1})
    xq, wq = a[rows].cpu().numpy(), w.cpu().numpy()
    ref = og.int8_gemm_ref(xq, sa[rows].cpu().numpy(), wq, sw.cpu().numpy(), b.cpu().numpy(),
                           acc=og.int8_matmul_exact(xq, wq))
    assert torch.equal(y[rows].cpu(), torch.from_numpy(ref).to(torch.bfloat16))


@pytest.mark.parametrize("m", [16, 256])
def test_ring_fp8_config_sizes_policy(m):
    """configs[3] at M = 16 and 256, K = N = 8192: the policy's kernel equals every ring instance bit for bit and the
    oracle on sampled rows."""
    g = torch.Generator(device=DEV).manual_seed(m)
    x = torch.randn(m, 8192, device=DEV, generator=g).bfloat16()
    w = torch.randn(8192, 8192, device=DEV, generator=g) * 0.02
    xq, sx = ops.quantize_act_fp8(x)
    wq, sw = ops.quantize_weight_fp8(w, "per_channel")
    y = ops.fp8_linear(xq, wq, sw, x_scale=sx, out_dtype=torch.bfloat16)
    for c in RINGS:
        assert torch.equal(y, ops.fp8_linear(xq, wq, sw, x_scale=sx, out_dtype=torch.bfloat16, config=c)), c
    rows = sorted({0, m // 2, m - 1})
    codes = lambda t: t.detach().cpu().view(torch.uint8).numpy()  # noqa: E731
    ref = og.fp8_gemm_ref(codes(xq[rows]), sx[rows].cpu().numpy(), codes(wq), sw.cpu().numpy())
    assert_close(y[rows].cpu(), ref, "bfloat16", what=f"fp8 ring policy m={m}")
