"""GPU parity of the 256 x 256 direct-to-LDS W8A8 kernel (fg_mm_big.hip): forced with tile_m=256 on ragged shapes
against the CPU oracle (INT8 accumulator and bf16/fp16 epilogue bit-exact, FP8 within the north-star bar), and at the
BASELINE configs' full sizes, where the C policy picks it by itself, against the 128 x 128 kernel on the same inputs
(same MFMA instruction and K order, so the results are bit-identical)."""
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
BIG = {"tile_m": 256}


def _i8(m, n, k, seed):
    x = torch.randn(m, k, generator=gen(seed)).numpy()
    w = (torch.randn(n, k, generator=gen(seed + 1)) * 0.05).numpy()
    xq, sx = og.quantize_int8_ref(x, "per_token")
    wq, sw = og.quantize_int8_ref(w, "per_channel")
    return xq, sx, wq, sw


@pytest.mark.parametrize("m,n,k", [(300, 520, 1024), (257, 517, 256), (1, 256, 128), (512, 512, 2048)])
def test_big_int8_exact_vs_oracle(m, n, k):
    xq, sx, wq, sw = _i8(m, n, k, seed=m + n + k)
    a, w = torch.from_numpy(xq).to(DEV), torch.from_numpy(wq).to(DEV)
    acc = ops.int8_gemm(a, None, w, None, out_dtype=torch.int32, config=BIG).cpu().numpy()
    ref_acc = og.int8_matmul_exact(xq, wq)
    assert np.array_equal(acc, ref_acc)
    b = torch.randn(n, generator=gen(9))
    ta, tb = torch.from_numpy(sx).to(DEV), torch.from_numpy(sw).to(DEV)
    y32 = ops.int8_gemm(a, ta, w, tb, b.to(DEV), out_dtype=torch.float32, config=BIG).cpu().numpy()
    ref32 = og.int8_gemm_ref(xq, sx, wq, sw, b.numpy(), acc=ref_acc)
    assert np.array_equal(y32, ref32)
    for odt in (torch.bfloat16, torch.float16):  # 16-bit epilogue (LDS transpose, 16-byte or ragged stores)
        y16 = ops.int8_gemm(a, ta, w, tb, b.to(DEV), out_dtype=odt, config=BIG).cpu()
        assert torch.equal(y16, torch.from_numpy(ref32).to(odt)), odt


@pytest.mark.parametrize("m,n,k", [(300, 520, 1024), (257, 517, 256), (64, 1024, 4096)])
def test_big_fp8_vs_oracle_and_small_tiles(m, n, k):
    x = torch.randn(m, k, generator=gen(m)).to(torch.bfloat16)
    w = torch.randn(n, k, generator=gen(n)) * 0.05
    xq, sx = og.quantize_fp8_ref(to_f32(x), "per_token")
    wq, sw = og.quantize_fp8_ref(w.numpy(), "per_channel")
    txq = torch.from_numpy(xq).view(torch.float8_e4m3fn).to(DEV)
    twq = torch.from_numpy(wq).view(torch.float8_e4m3fn).to(DEV)
    tsx, tsw = torch.from_numpy(sx).to(DEV), torch.from_numpy(sw).to(DEV)
    b = (torch.randn(n, generator=gen(4)) * 0.1).to(torch.bfloat16).to(DEV)
    for odt in (torch.bfloat16, torch.float16, torch.float32):
        y = ops.fp8_linear(txq, twq, tsw, b, x_scale=tsx, out_dtype=odt, config=BIG)
        y128 = ops.fp8_linear(txq, twq, tsw, b, x_scale=tsx, out_dtype=odt, config={"tile_m": 128})
        assert torch.equal(y, y128), odt
    ref = og.fp8_gemm_ref(xq, sx, wq, sw, to_f32(b.cpu()))
    assert_close(y.cpu(), ref, "float32", what=f"fp8 big m={m}")


def test_big_rejects_unsupported_shapes():
    a = torch.zeros(512, 1000, dtype=torch.int8, device=DEV)
    w = torch.zeros(512, 1000, dtype=torch.int8, device=DEV)
    with pytest.raises(_lib.KernelLaunchError, match="tile_m=256"):
        ops.int8_gemm(a, None, w, None, out_dtype=torch.int32, config=BIG)
    # the automatic policy falls back to the 128 x 128 kernel for such K
    assert ops.int8_gemm(a, None, w, None, out_dtype=torch.int32).abs().sum().item() == 0


@pytest.mark.parametrize("k,n", [(8192, 10240), (28672, 8192)])
def test_big_int8_full_size_matches_128_tiles(k, n):
    """configs[4] at M=4096: the automatic policy (256 x 256 kernel) equals the 128 x 128 kernel bit for bit."""
    g = torch.Generator(device=DEV).manual_seed(k + n)
    a = torch.randint(-127, 128, (4096, k), dtype=torch.int8, device=DEV, generator=g)
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=DEV, generator=g)
    y = ops.int8_gemm(a, None, w, None, out_dtype=torch.int32)
    y128 = ops.int8_gemm(a, None, w, None, out_dtype=torch.int32, config={"tile_m": 128})
    assert torch.equal(y, y128)
    # spot-check a few rows against the exact oracle
    rows = [0, 1777, 4095]
    ref = og.int8_matmul_exact(a[rows].cpu().numpy(), w.cpu().numpy())
    assert np.array_equal(y[rows].cpu().numpy(), ref)


@pytest.mark.parametrize("n", [10240, 10203])
def test_big_int8_wide_tiles_bf16(n):
    """M=4096, N~10240: 640 tiles of 256 x 256 would fill 2.5 rounds of 256 CUs, so the policy runs 256 x 320 tiles
    (2 rounds) for 16-bit outputs; the bf16 result equals the 128 x 128 kernel's bit for bit (same int32 accumulators,
    same epilogue order), the ragged last tile included, and matches the oracle on sampled rows."""
    g = torch.Generator(device=DEV).manual_seed(n)
    a = torch.randint(-127, 128, (4096, 1024), dtype=torch.int8, device=DEV, generator=g)
    w = torch.randint(-127, 128, (n, 1024), dtype=torch.int8, device=DEV, generator=g)
    sa = torch.rand(4096, device=DEV, generator=g) * 0.01 + 0.001
    sw = torch.rand(n, device=DEV, generator=g) * 0.01 + 0.001
    b = torch.randn(n, device=DEV, generator=g)
    y = ops.int8_gemm(a, sa, w, sw, b, out_dtype=torch.bfloat16)
    y128 = ops.int8_gemm(a, sa, w, sw, b, out_dtype=torch.bfloat16, config={"tile_m": 128})
    assert torch.equal(y, y128)
    rows = [0, 1023, 2050, 4095]
    xq, wq = a[rows].cpu().numpy(), w.cpu().numpy()
    ref = og.int8_gemm_ref(xq, sa[rows].cpu().numpy(), wq, sw.cpu().numpy(), b.cpu().numpy(),
                           acc=og.int8_matmul_exact(xq, wq))
    assert torch.equal(y[rows].cpu(), torch.from_numpy(ref).to(torch.bfloat16))


def test_big_fp8_full_size_matches_128_tiles():
    """configs[3] at M=4096, K=N=8192 with bf16 output and per-token x per-channel scales."""
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(4096, 8192, device=DEV, generator=g).bfloat16()
    w = torch.randn(8192, 8192, device=DEV, generator=g) * 0.02
    xq, sx = ops.quantize_act_fp8(x)
    wq, sw = ops.quantize_weight_fp8(w, "per_channel")
    y = ops.fp8_linear(xq, wq, sw, x_scale=sx, out_dtype=torch.bfloat16)
    y128 = ops.fp8_linear(xq, wq, sw, x_scale=sx, out_dtype=torch.bfloat16, config={"tile_m": 128})
    assert torch.equal(y, y128)
    rows = [0, 2049, 4095]
    ref = og.fp8_gemm_ref(ops_codes(xq[rows]), sx[rows].cpu().numpy(), ops_codes(wq), sw.cpu().numpy())
    assert_close(y[rows].cpu(), ref, "bfloat16", what="fp8 full-size rows")


@pytest.mark.parametrize("m,n,cfg", [(192, 57344, BIG), (300, 28672, BIG), (640, 14336, BIG),
                                     (160, 10240, {"tile_m": 64, "tile_n": 128})])
def test_policy_mid_m_kernels(m, n, cfg):
    """129..1023 rows: the 256-row kernel once its tiles number 5/8 of the CUs (224 tiles at M = 192 / 300, 168 at
    M = 640) and 64 x 128 ring tiles where they fit one per CU (240 at M = 160, N = 10240).  The policy's INT8 and FP8
    results equal the named instance's bit for bit and match the oracle on sampled rows (bf16 output, per-token x
    per-channel scales, bias)."""
    k = 512
    g = torch.Generator(device=DEV).manual_seed(m + n)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=DEV, generator=g)
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=DEV, generator=g)
    sa = torch.rand(m, device=DEV, generator=g) * 0.01 + 0.001
    sw = torch.rand(n, device=DEV, generator=g) * 0.01 + 0.001
    b = torch.randn(n, device=DEV, generator=g)
    y = ops.int8_gemm(a, sa, w, sw, b, out_dtype=torch.bfloat16)
    assert torch.equal(y, ops.int8_gemm(a, sa, w, sw, b, out_dtype=torch.bfloat16, config=cfg))
    rows = sorted({0, m // 2, m - 1})
    xq, wq = a[rows].cpu().numpy(), w.cpu().numpy()
    ref = og.int8_gemm_ref(xq, sa[rows].cpu().numpy(), wq, sw.cpu().numpy(), b.cpu().numpy(),
                           acc=og.int8_matmul_exact(xq, wq))
    assert torch.equal(y[rows].cpu(), torch.from_numpy(ref).to(torch.bfloat16))
    x = torch.randn(m, k, device=DEV, generator=g).bfloat16()
    xf, sx = ops.quantize_act_fp8(x)
    wf, swf = ops.quantize_weight_fp8(torch.randn(n, k, device=DEV, generator=g) * 0.02, "per_channel")
    yf = ops.fp8_linear(xf, wf, swf, x_scale=sx, out_dtype=torch.bfloat16)
    assert torch.equal(yf, ops.fp8_linear(xf, wf, swf, x_scale=sx, out_dtype=torch.bfloat16, config=cfg))
    ref = og.fp8_gemm_ref(ops_codes(xf[rows]), sx[rows].cpu().numpy(), ops_codes(wf), swf.cpu().numpy())
    assert_close(yf[rows].cpu(), ref, "bfloat16", what=f"fp8 policy m={m} n={n}")


def ops_codes(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.uint8).numpy()
