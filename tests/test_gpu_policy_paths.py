"""GPU parity of the kernels the automatic per-shape policy picks at the configs' full sizes, where no other test
forces them: W4A16 at 33..64 rows over the Llama-3-8B linears (the LDS-ring kernel plus its split-K reduce; the
64-row dequantise-to-LDS prefill tiles, forced, beside it) and at 13..32 rows (the LDS-ring kernel; the skinny MFMA
kernel, forced, beside it), W8A16 at 33..64 rows, W4A16 at 4 rows over gate+up (skinny MFMA kernel), 256-row prefill tiles with fp16 x,
and INT8 W8A8 at configs[4]'s (K, N) = (8192, 57344) and (28672, 8192) for M = 1 and 4096.

Bars: W4/W8A16 within max|y - ref| / max|ref| <= 1e-2 of the fp32 oracle plus the reference's compare() rule;
INT8 int32 accumulators and the fp32 -> bf16 epilogue bit-exact on sampled rows.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from forge_amd import layouts as L
from forge_amd import ops_gemm as ops
from oracle import gemm as og
from oracle import w4 as ow
from tests._util import assert_close, gen, oracle_packed, to_f32, w4_parts, x_act

pytestmark = pytest.mark.gpu
DEV = "cuda"
ODT = {torch.bfloat16: "bfloat16", torch.float16: "float16"}
LLAMA = {"qkv": (4096, 6144), "o_proj": (4096, 4096), "gate_up": (4096, 28672), "down": (14336, 4096)}  # (K, N)


def _rows_oracle(xs: list[torch.Tensor], packed: dict) -> list[np.ndarray]:
    """One oracle GEMM over the stacked rows of every case (rows are independent), split back per case."""
    ref = og.w4a16_gemm_ref(np.concatenate([to_f32(x) for x in xs]), packed)
    out, r0 = [], 0
    for x in xs:
        out.append(ref[r0:r0 + x.shape[0]])
        r0 += x.shape[0]
    return out


@pytest.mark.parametrize("shape", sorted(LLAMA))
def test_w4_policy_33_to_64_rows_full_size(shape):
    """M in {33, 48, 64}: the policy runs the LDS-ring kernel (K splits summed by a second launch), forcing
    impl=prefill the 64-row prefill tiles with their split-K reduce; both against the oracle, the policy's result
    reproducible run to run."""
    k, n = LLAMA[shape]
    q, s, z = w4_parts(n, k, 128, False, seed=k + n)
    p = L.pack_w4(q, s, z, 128).to(DEV)
    cases = [(33, torch.bfloat16, True), (48, torch.float16, False), (64, torch.bfloat16, False),
             (64, torch.float16, True)]
    xs = [x_act(m, k, xdt, seed=m + i) for i, (m, xdt, _) in enumerate(cases)]
    refs = _rows_oracle(xs, oracle_packed(q, s, z, 128))
    for (m, xdt, has_b), x, ref in zip(cases, xs, refs):
        b = (torch.randn(n, generator=gen(m)) * 0.5).to(xdt) if has_b else None
        bd = None if b is None else b.to(DEV)
        y = ops.w4a16_linear(x.to(DEV), p, bd)
        assert ops.last_path("w4a16_linear") == "hip"
        r = ref if b is None else (ref + to_f32(b)).astype(np.float32)
        assert_close(y.cpu(), r, ODT[xdt], what=f"w4 policy {shape} m={m}")
        assert torch.equal(y, ops.w4a16_linear(x.to(DEV), p, bd)), f"{shape} m={m}: policy not reproducible"
        yf = ops.w4a16_linear(x.to(DEV), p, bd, config={"impl": "prefill"})
        assert_close(yf.cpu(), r, ODT[xdt], what=f"w4 forced prefill {shape} m={m}")


@pytest.mark.parametrize("shape", ["qkv", "o_proj", "gate_up"])
def test_w4_policy_13_to_32_rows_full_size(shape):
    """17..32 rows (13..16 over gate+up's 28672 channels): the policy runs the LDS-ring kernel on portable_row
    weights; forcing impl=mfma runs the skinny kernel.  Both against the oracle, the policy's result reproducible."""
    k, n = LLAMA[shape]
    q, s_, z = w4_parts(n, k, 128, False, seed=k + n + 1)
    p = L.pack_w4(q, s_, z, 128).to(DEV)
    cases = [(17, torch.bfloat16, True), (24, torch.float16, False), (32, torch.bfloat16, False)]
    if shape == "gate_up":
        cases.append((13, torch.float16, True))
    xs = [x_act(m, k, xdt, seed=m + 5 * i) for i, (m, xdt, _) in enumerate(cases)]
    refs = _rows_oracle(xs, oracle_packed(q, s_, z, 128))
    for (m, xdt, has_b), x, ref in zip(cases, xs, refs):
        b = (torch.randn(n, generator=gen(m + 1)) * 0.5).to(xdt) if has_b else None
        bd = None if b is None else b.to(DEV)
        y = ops.w4a16_linear(x.to(DEV), p, bd)
        assert ops.last_path("w4a16_linear") == "hip"
        r = ref if b is None else (ref + to_f32(b)).astype(np.float32)
        assert_close(y.cpu(), r, ODT[xdt], what=f"w4 policy {shape} m={m}")
        assert torch.equal(y, ops.w4a16_linear(x.to(DEV), p, bd)), f"{shape} m={m}: policy not reproducible"
        yf = ops.w4a16_linear(x.to(DEV), p, bd, config={"impl": "mfma"})
        assert_close(yf.cpu(), r, ODT[xdt], what=f"w4 forced skinny {shape} m={m}")


def test_w4_policy_64_rows_symmetric_qkv():
    k, n = LLAMA["qkv"]
    q, s, z = w4_parts(n, k, 128, True, seed=3)
    p = L.pack_w4(q, s, z, 128).to(DEV)
    x = x_act(64, k, torch.bfloat16, seed=4)
    y = ops.w4a16_linear(x.to(DEV), p)
    assert_close(y.cpu(), og.w4a16_gemm_ref(to_f32(x), oracle_packed(q, s, z, 128)), "bfloat16", what="sym m=64")


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_w4_policy_4_rows_gate_up(xdt):
    """M=4 over gate+up (4096 x 28672): the skinny MFMA kernel (3..4 rows over weights above 4096 x 4096)."""
    k, n = LLAMA["gate_up"]
    q, s, z = w4_parts(n, k, 128, False, seed=7)
    p = L.pack_w4(q, s, z, 128).to(DEV)
    x = x_act(4, k, xdt, seed=8)
    b = (torch.randn(n, generator=gen(9)) * 0.5).to(xdt)
    y = ops.w4a16_linear(x.to(DEV), p, b.to(DEV))
    ref = og.w4a16_gemm_ref(to_f32(x), oracle_packed(q, s, z, 128), to_f32(b))
    assert_close(y.cpu(), ref, ODT[xdt], what="gate_up m=4")


@pytest.mark.parametrize("m,n,k,gs,xdt,sdt", [
    (2048, 8192, 1024, 128, torch.float16, torch.float16),   # 256 tiles of 256 x 256: the all-rounder's 256-row tiles
    (2048, 8192, 512, -1, torch.bfloat16, torch.float32),    # the same with fp32 scales (plain K loop), one group
])
def test_w4_prefill_256_row_tiles(m, n, k, gs, xdt, sdt):
    """The all-round prefill kernel (tile_n = 64 forces it; the policy runs the ping-pong kernel on these shapes)."""
    q, s, z = w4_parts(n, k, gs, False, seed=m + k, scale_dtype=sdt)
    p = L.pack_w4(q, s, z, gs).to(DEV)
    x = x_act(m, k, xdt, seed=k)
    b = (torch.randn(n, generator=gen(k)) * 0.5).to(xdt)
    y = ops.w4a16_linear(x.to(DEV), p, b.to(DEV), config={"impl": "prefill", "tile_n": 64})
    assert ops.last_kernel().startswith("w4_big_kernel<256"), ops.last_kernel()
    ref = og.w4a16_gemm_ref(to_f32(x), oracle_packed(q, s, z, gs), to_f32(b))
    assert_close(y.cpu(), ref, ODT[xdt], what=f"prefill 256-row m={m} n={n} k={k}")


@pytest.mark.parametrize("shape", ["qkv", "down"])
def test_w8a16_policy_64_rows_prefill_kernel(shape):
    """W8A16 at M = 64 with group 64 (the skinny kernel needs groups of 128): the prefill kernel's 64-row tiles."""
    k, n = LLAMA[shape]
    g = gen(k + n)
    q = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand(n, k // 64, generator=g) * 0.018 + 0.002).half()
    p = L.pack_w8(q, s, 64).to(DEV)
    x = x_act(64, k, torch.bfloat16, seed=5)
    y = ops.w8a16_linear(x.to(DEV), p)
    ref = og.w8a16_gemm_ref(to_f32(x), og.pack_w8(q.numpy(), s.float().numpy(), 64))
    assert_close(y.cpu(), ref, "bfloat16", what=f"w8a16 m=64 {shape}")
    yf = ops.w8a16_linear(x.to(DEV), p, config={"impl": "prefill"})
    assert torch.equal(y, yf)


def _int8_operands(m, n, k, seed):
    gd = torch.Generator(device=DEV).manual_seed(seed)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=DEV, generator=gd)
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=DEV, generator=gd)
    sa = torch.rand(m, device=DEV, generator=gd) * 0.01 + 0.001
    sw = torch.rand(n, device=DEV, generator=gd) * 0.01 + 0.001
    return a, w, sa, sw


@pytest.mark.parametrize("m,k,n", [(4096, 8192, 57344), (1, 8192, 57344), (1, 28672, 8192), (64, 8192, 57344)])
def test_int8_configs4_shapes_exact(m, k, n):
    """configs[4] shapes the other tests leave out, through the policy: raw int32 accumulator and bf16 epilogue
    bit-exact against the oracle on sampled rows (all N columns)."""
    a, w, sa, sw = _int8_operands(m, n, k, seed=m + k + n)
    acc = ops.int8_gemm(a, None, w, None, out_dtype=torch.int32)
    y = ops.int8_gemm(a, sa, w, sw, None, out_dtype=torch.bfloat16)
    rows = sorted({0, m // 3, (2 * m) // 3, m - 1})
    xq, wq = a[rows].cpu().numpy(), w.cpu().numpy()
    ref_acc = og.int8_matmul_exact(xq, wq)
    assert np.array_equal(acc[rows].cpu().numpy(), ref_acc)
    ref = og.int8_gemm_ref(xq, sa[rows].cpu().numpy(), wq, sw.cpu().numpy(), None, acc=ref_acc)
    assert torch.equal(y[rows].cpu(), torch.from_numpy(ref).to(torch.bfloat16))


# ---------------------------------------------------------------------------------------------- configs[2] prefill
_PREFILL_CACHE: dict = {}


def _prefill_weights(shape: str, bits: int):
    """One weight per (shape, bits) for every M of the prefill cells: the packed GPU copy and the oracle's fp32
    dequantised ``[N, K]`` (rows of x times its transpose are the oracle's rows of y)."""
    key = (shape, bits)
    if key not in _PREFILL_CACHE:
        if any(sh != shape for sh, _ in _PREFILL_CACHE):
            _PREFILL_CACHE.clear()  # one shape at a time: gate+up's dequantised oracle weight is 470 MB per format
        k, n = LLAMA[shape]
        if bits == 4:
            q, s, z = w4_parts(n, k, 128, False, seed=2 * k + n)
            packed = L.pack_w4(q, s, z, 128).to(DEV)
            dense = ow.dequantize_parts(q.numpy(), s.float().numpy(), z.numpy(), 128)
        else:
            g = gen(3 * k + n)
            q = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
            s = (torch.rand(n, k // 128, generator=g) * 0.018 + 0.002).half()
            packed = L.pack_w8(q, s, 128).to(DEV)
            dense = og.dequantize_w8(og.pack_w8(q.numpy(), s.float().numpy(), 128))
        _PREFILL_CACHE[key] = (packed, dense)
    return _PREFILL_CACHE[key]


PREFILL_CELLS = [(m, sh) for sh in ("qkv", "o_proj", "gate_up", "down") for m in (512, 2048, 8192)]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m,shape", PREFILL_CELLS)
def test_prefill_policy_configs2_cells(m, shape, bits):
    """M in {512, 2048, 8192} on the four Llama-3-8B shapes through the automatic policy (bf16 x ~ N(0,1),
    group 128; W4 asymmetric with zero-points U{6..9}, W8A16 symmetric int8).  Rows sampled from the first, middle
    and last row tiles are checked against the oracle over all N columns, within the north-star bar plus compare();
    the result is reproducible run to run."""
    k, n = LLAMA[shape]
    packed, dense = _prefill_weights(shape, bits)
    x = x_act(m, k, torch.bfloat16, seed=m + k + n + bits)
    xd = x.to(DEV)
    op = ops.w4a16_linear if bits == 4 else ops.w8a16_linear
    y = op(xd, packed)
    assert ops.last_path("w4a16_linear" if bits == 4 else "w8a16_linear") == "hip"
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    rows = sorted({0, 1, 127, 128, m // 2 + 5, m - 129, m - 2, m - 1})
    ref = (to_f32(x[rows]) @ dense.T).astype(np.float32)
    assert_close(y[rows].cpu(), ref, "bfloat16", what=f"w{bits} prefill {shape} m={m}")
    assert torch.equal(y, op(xd, packed)), f"w{bits} {shape} m={m}: not reproducible"
