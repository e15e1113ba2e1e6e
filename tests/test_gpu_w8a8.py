"""GPU parity of the W8A8 path through the C ABI: INT8 GEMM (exact int32 accumulator, exact fp32 epilogue), FP8
e4m3fn GEMM (all three scale modes), and the per-token / block quantisers, against the CPU oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from forge_amd import ops_gemm as ops
from oracle import gemm as og
from tests._util import assert_close, fp8_codes, gen, to_f32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _int8_operands(m, n, k, seed):
    x = torch.randn(m, k, generator=gen(seed)).numpy()
    w = (torch.randn(n, k, generator=gen(seed + 1)) * 0.05).numpy()
    xq, sx = og.quantize_int8_ref(x, "per_token")
    wq, sw = og.quantize_int8_ref(w, "per_channel")
    return xq, sx, wq, sw


# ------------------------------------------------------------------------------------------------ INT8
@pytest.mark.parametrize("m", [1, 16, 100, 513])
@pytest.mark.parametrize("n,k", [(4096, 4096), (777, 1000)])
def test_int8_gemm_exact(m, n, k):
    """int32 accumulator bit-exact; the fp32 epilogue equals the oracle bit for bit (torch.equal bar of
    tests_gpu/test_kernels_gemm_fp8_int8.py:106-117)."""
    xq, sx, wq, sw = _int8_operands(m, n, k, seed=m + n)
    a, w = torch.from_numpy(xq).to(DEV), torch.from_numpy(wq).to(DEV)
    acc = ops.int8_gemm(a, None, w, None, out_dtype=torch.int32).cpu().numpy()
    ref_acc = og.int8_matmul_exact(xq, wq)
    assert np.array_equal(acc, ref_acc)
    b = torch.randn(n, generator=gen(7))
    y = ops.int8_gemm(a, torch.from_numpy(sx).to(DEV), w, torch.from_numpy(sw).to(DEV), b.to(DEV),
                      out_dtype=torch.float32).cpu().numpy()
    assert np.array_equal(y, og.int8_gemm_ref(xq, sx, wq, sw, b.numpy(), acc=ref_acc))


@pytest.mark.parametrize("m", [1, 2])
@pytest.mark.parametrize("n,k", [(4096, 4096), (776, 1008), (1024, 16), (264, 28672), (8, 8192)])
def test_int8_gemv_exact(m, n, k):
    """The decode GEMV (the policy's choice for 1..2 rows, and forced with tile_m=1): int32 accumulator and fp32 /
    bf16 epilogue bit-exact against the oracle, with and without bias."""
    xq, sx, wq, sw = _int8_operands(m, n, k, seed=m + n + k)
    a, w = torch.from_numpy(xq).to(DEV), torch.from_numpy(wq).to(DEV)
    ref_acc = og.int8_matmul_exact(xq, wq)
    for cfg in (None, {"tile_m": 1}):
        acc = ops.int8_gemm(a, None, w, None, out_dtype=torch.int32, config=cfg).cpu().numpy()
        assert np.array_equal(acc, ref_acc), cfg
    b = torch.randn(n, generator=gen(9))
    y = ops.int8_gemm(a, torch.from_numpy(sx).to(DEV), w, torch.from_numpy(sw).to(DEV), b.to(DEV),
                      out_dtype=torch.float32).cpu().numpy()
    assert np.array_equal(y, og.int8_gemm_ref(xq, sx, wq, sw, b.numpy(), acc=ref_acc))
    y16 = ops.int8_gemm(a, torch.from_numpy(sx).to(DEV), w, torch.from_numpy(sw).to(DEV), out_dtype=torch.bfloat16)
    ref16 = torch.from_numpy(og.int8_gemm_ref(xq, sx, wq, sw, acc=ref_acc)).bfloat16()
    assert torch.equal(y16.cpu(), ref16)


def test_int8_gemv_extremes_and_rejects():
    """127 / -128 everywhere over K = 28672 (|acc| up to 4.7e8, still exact in int32); tile_m=1 rejects 3 rows."""
    k, n = 28672, 64
    xq = np.full((2, k), -128, dtype=np.int8)
    xq[1, ::2] = 127
    wq = np.full((n, k), 127, dtype=np.int8)
    wq[::3] = -128
    a, w = torch.from_numpy(xq).to(DEV), torch.from_numpy(wq).to(DEV)
    acc = ops.int8_gemm(a, None, w, None, out_dtype=torch.int32, config={"tile_m": 1}).cpu().numpy()
    assert np.array_equal(acc, og.int8_matmul_exact(xq, wq))
    from forge_amd import _lib
    with pytest.raises(_lib.KernelLaunchError, match="tile_m=1"):
        ops.int8_gemm(torch.zeros(3, k, dtype=torch.int8, device=DEV), None, w, None, out_dtype=torch.int32,
                      config={"tile_m": 1})


@pytest.mark.parametrize("m", [0, 1, 16, 100])
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_int8_linear_end_to_end(m, xdt):
    n, k = 777, 1000
    x = torch.randn(m, k, generator=gen(3)).to(xdt)
    w = (torch.randn(n, k, generator=gen(4)) * 0.05)
    wq, sw = og.quantize_int8_ref(w.numpy(), "per_channel")
    y = ops.int8_linear(x.to(DEV), torch.from_numpy(wq).to(DEV), torch.from_numpy(sw).to(DEV))
    assert ops.last_path("int8_linear") == "hip" and y.dtype == xdt and y.shape == (m, n)
    if m == 0:
        return
    xr, sr = og.quantize_int8_ref(to_f32(x), "per_token")
    assert_close(y.cpu(), og.int8_gemm_ref(xr, sr, wq, sw), "float16" if xdt == torch.float16 else "bfloat16")


@pytest.mark.parametrize("m,k", [(1, 1000), (16, 4096), (100, 1000), (513, 4096)])
def test_int8_quantiser_bit_exact(m, k):
    x = torch.randn(m, k, generator=gen(m)).to(torch.float16)
    q, s = ops.quantize_act_int8(x.to(DEV))
    qr, sr = og.quantize_int8_ref(to_f32(x), "per_token")
    assert np.array_equal(s.cpu().numpy(), sr)
    assert np.array_equal(q.cpu().numpy(), qr)


def test_int8_quantiser_ties_zero_rows_nan():
    x = torch.tensor([[2.5, 127.0, -2.5, 0.5, 1.5, -126.5], [0.0] * 6, [1.0, float("nan"), 300.0, -3.0, 0.0, 2.0]])
    q, s = ops.quantize_act_int8(x.to(DEV))
    qr, sr = og.quantize_int8_ref(x.numpy(), "per_token")
    assert np.array_equal(s.cpu().numpy(), sr) and np.array_equal(q.cpu().numpy(), qr)
    assert q[0].tolist() == [2, 127, -2, 0, 2, -126]


# ------------------------------------------------------------------------------------------------ FP8
@pytest.mark.parametrize("gx,gw", [("per_tensor", "per_tensor"), ("per_token", "per_channel"), ("block", "block2d")])
@pytest.mark.parametrize("m", [0, 1, 7, 64, 300])
@pytest.mark.parametrize("n,k", [(4096, 4096), (1000, 2056), (256, 777)])
def test_fp8_gemm_matches_oracle(gx, gw, m, n, k):
    x = torch.randn(m, k, generator=gen(m + k)).to(torch.bfloat16)
    w = torch.randn(n, k, generator=gen(n)) * 0.05
    xq, sx = og.quantize_fp8_ref(to_f32(x), gx)
    wq, sw = og.quantize_fp8_ref(w.numpy(), gw)
    txq = torch.from_numpy(xq).view(torch.float8_e4m3fn).to(DEV)
    twq = torch.from_numpy(wq).view(torch.float8_e4m3fn).to(DEV)
    y = ops.fp8_linear(txq, twq, torch.from_numpy(sw).to(DEV), x_scale=torch.from_numpy(sx).to(DEV),
                       out_dtype=torch.bfloat16)
    assert ops.last_path("fp8_linear") == "hip" and y.shape == (m, n)
    if m:
        assert_close(y.cpu(), og.fp8_gemm_ref(xq, sx, wq, sw), "bfloat16", what=f"fp8 {gx}/{gw} m={m}")


def test_fp8_gemm_is_bit_reproducible_and_bias():
    x = torch.randn(256, 4096, generator=gen(1)).to(torch.bfloat16)
    w = torch.randn(4096, 4096, generator=gen(2)) * 0.05
    wq, sw = og.quantize_fp8_ref(w.numpy(), "per_channel")
    twq, tsw = torch.from_numpy(wq).view(torch.float8_e4m3fn).to(DEV), torch.from_numpy(sw).to(DEV)
    b = torch.randn(4096, generator=gen(3)).to(torch.bfloat16)
    outs = [ops.fp8_linear(x.to(DEV), twq, tsw, b.to(DEV)) for _ in range(5)]
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    xq, sx = og.quantize_fp8_ref(to_f32(x), "per_token")
    assert_close(outs[0].cpu(), og.fp8_gemm_ref(xq, sx, wq, sw, to_f32(b)), "bfloat16", what="fp8 e2e + bias")


@pytest.mark.parametrize("gran,block", [("per_token", 128), ("per_tensor", 128), ("block", 128), ("block2d", 128),
                                        ("block", 64)])
@pytest.mark.parametrize("m,k", [(1, 64), (33, 1000), (300, 4096)])
def test_fp8_quantiser_codes_bit_exact(gran, block, m, k):
    x = (torch.randn(m, k, generator=gen(m * k)) * 3).to(torch.bfloat16)
    x[0, : min(k, 5)] = torch.tensor([2 ** -12, -2 ** -10, 3 * 2 ** -11, 0.0, 1e-30])[: min(k, 5)].to(torch.bfloat16)
    q, s = ops.quantize_act_fp8(x.to(DEV), granularity=gran, block=block)
    qr, sr = og.quantize_fp8_ref(to_f32(x), gran, block=block)
    assert np.array_equal(s.cpu().numpy().reshape(sr.shape), sr)
    assert np.array_equal(fp8_codes(q), qr)


def test_fp8_quantiser_edge_cases():
    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    x[1] = 1e4
    x[2, 0] = 1e-6
    q, s = ops.quantize_act_fp8(x.to(DEV))
    qr, sr = og.quantize_fp8_ref(to_f32(x), "per_token")
    assert np.array_equal(fp8_codes(q), qr) and np.array_equal(s.cpu().numpy(), sr)
    assert s[0].item() == 1.0 and q[1].float().abs().max().item() == 448.0
    # static scale smaller than needed saturates (never NaN)
    big = torch.tensor([[1000.0, -1000.0, 1.0]])
    qs, _ = ops.quantize_act_fp8(big.to(DEV), granularity="per_tensor", scale=torch.tensor([1.0]))
    assert qs.float().cpu().tolist() == [[448.0, -448.0, 1.0]]
    xn = torch.randn(2, 128, generator=gen(5)).to(torch.bfloat16)
    xn[0, 5] = float("nan")
    qn, sn = ops.quantize_act_fp8(xn.to(DEV))
    qnr, snr = og.quantize_fp8_ref(to_f32(xn), "per_token")
    assert np.array_equal(sn.cpu().numpy(), snr)
    assert np.array_equal(fp8_codes(qn), qnr) and torch.isfinite(qn[1].float()).all()  # NaN code 0x7F / 0xFF too


@pytest.mark.parametrize("k", [64, 1000, 4096, 12288])
def test_fused_rmsnorm_fp8_quantiser(k):
    """Against the float64 definition y = x / sqrt(mean(x^2) + eps) * w: the kernel sums x^2 in another order than
    the CPU oracle, so its scale may sit a few fp32 ulps away and a code may land on the other side of a rounding
    midpoint.  Bars: scale within 2e-6 relative of amax(y64) / 448; every code the correct rounding of y64 / s for the
    kernel's own s, except where that value lies within 8e-6 relative of a midpoint between two codes, and then one
    of those two; codes equal to the oracle's wherever no midpoint is that close."""
    x = (torch.randn(33, k, generator=gen(k)) * 3).to(torch.bfloat16)
    wt = (torch.rand(k, generator=gen(k + 1)) + 0.5).to(torch.bfloat16)
    x[7] = 0  # a zero row: scale 1, codes 0
    q, s = ops.quantize_act_fp8(x.to(DEV), rms_weight=wt.to(DEV), rms_eps=1e-6)
    qr, sr, _ = og.rmsnorm_act_quant_fp8_ref(to_f32(x), to_f32(wt), 1e-6)
    x64, w64 = to_f32(x).astype(np.float64), to_f32(wt).astype(np.float64)
    y64 = x64 / np.sqrt((x64 * x64).mean(-1, keepdims=True) + 1e-6) * w64
    s_gpu = s.cpu().numpy().astype(np.float64)
    amax = np.abs(y64).max(-1)
    s64 = np.where(amax > 0, amax / 448.0, 1.0)
    assert np.all(np.abs(s_gpu - s64) <= 2e-6 * s64), np.abs(s_gpu / s64 - 1).max()
    assert s_gpu[7] == 1.0 and np.all(fp8_codes(q)[7] == 0)
    v = np.clip(y64 / s_gpu[:, None], -448.0, 448.0)
    codes, exact = fp8_codes(q), og.e4m3_encode(v.astype(np.float32))
    # the rounding boundary nearest to |v|: the midpoint between the correct code and its neighbour on v's side
    a, c = np.abs(v), (exact & 0x7F).astype(np.int64)
    dc = og.e4m3_decode(c.astype(np.uint8)).astype(np.float64)
    nb = np.clip(np.where(a > dc, c + 1, c - 1), 0, 0x7E)
    mid = (dc + og.e4m3_decode(nb.astype(np.uint8)).astype(np.float64)) / 2
    near = np.abs(a - mid) <= 8e-6 * a
    diff = codes != exact
    assert np.all(near[diff]), f"{int((diff & ~near).sum())} codes off the correct rounding"
    dq = og.e4m3_decode(codes).astype(np.float64)
    assert np.all(np.abs(dq[diff] - v[diff]) <= np.abs(og.e4m3_decode(exact).astype(np.float64)[diff] - v[diff]) * 1.0001
                  + 8e-6 * np.abs(v[diff]))  # the other side of the same midpoint
    assert np.array_equal(codes[~near], qr[~near])
