"""Pins of the CPU oracle (oracle/): each oracle function is checked against something independent of it --
closed forms in float64, brute force, torch's own casts, the C restatement, and the known answers of the reference's
tests (forge-llm tests/test_kernels_gemm_refs.py, tests/test_kernels_gemm_layouts.py).  No GPU, no HIP calls."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import gemm as og
from oracle import w4 as ow


def rnd(*shape, seed=0, scale=1.0):
    return (torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale).numpy()


# ------------------------------------------------------------------------------------------- layout id / nibbles
def test_layout_ids_match_reference_signature_hash():
    # ids recomputed from the reference's storage signature (forge/kernels/layouts/layout.py:167-198)
    assert ow.layout_id(4) == "w4.portable_row.v1-73e10e"
    assert ow.layout_id(8) == "w8.portable_row.v1-db2653"


def test_pack_nibbles_brute_force():
    rng = np.random.default_rng(0)
    nib = rng.integers(0, 16, size=(5, 7, 8), dtype=np.uint8)
    words = ow.pack_nibbles_int32(nib)
    for idx in np.ndindex(5, 7):
        v = sum(int(nib[idx][j]) << (4 * j) for j in range(8))
        v = v - (1 << 32) if v >= 1 << 31 else v
        assert int(words[idx]) == v
    assert np.array_equal(ow.unpack_nibbles_int32(words), nib)
    # top nibble 15 sets the sign bit: two's complement wrap, still exact
    assert int(ow.pack_nibbles_int32(np.full(8, 15, np.uint8))) == -1


def test_pack_w4_brute_force_positions_and_padding():
    n, k, gs = 3, 21, 8  # K not a multiple of 8 -> 3 pad columns
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    g = ow.num_groups(k, gs)
    s = rng.random((n, g), dtype=np.float32) + 0.5
    z = rng.integers(0, 16, size=(n, g), dtype=np.uint8)
    p = ow.pack_w4(q, s, z, gs)
    assert p["qweight"].shape == (n, 3) and p["scales"].shape == (g, n) and p["zeros"].shape == (g, 1)
    for i in range(n):
        for kk in range(24):
            word = int(p["qweight"][i, kk // 8]) & 0xFFFFFFFF
            got = (word >> (4 * (kk % 8))) & 0xF
            want = int(q[i, kk]) if kk < k else int(z[i, min(kk // gs, g - 1)])  # pads carry the zero-point
            assert got == want
    for gg in range(g):
        zw = int(p["zeros"][gg, 0]) & 0xFFFFFFFF
        for i in range(n):
            assert (zw >> (4 * i)) & 0xF == z[i, gg]
    assert np.array_equal(p["scales"], s.T)


@pytest.mark.parametrize("n", [1, 7, 63, 64, 65, 130])
@pytest.mark.parametrize("k", [8, 16, 33, 100, 128, 257])
@pytest.mark.parametrize("gs", [-1, 16, 64])
@pytest.mark.parametrize("sym", [True, False])
def test_pack_unpack_identity_property_matrix(n, k, gs, sym):
    """Reference property matrix (tests/test_kernels_gemm_layouts.py:136-151), portable layout."""
    rng = np.random.default_rng(n * 1000 + k)
    g = ow.num_groups(k, gs)
    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    s = rng.random((n, g), dtype=np.float32)
    z = None if sym else rng.integers(0, 16, size=(n, g), dtype=np.uint8)
    q2, s2, z2 = ow.unpack_w4(ow.pack_w4(q, s, z, gs))
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    assert (z is None and z2 is None) or np.array_equal(z, z2)


def test_dequantize_parts_closed_form_float64_and_special_cases():
    rng = np.random.default_rng(2)
    n, k, gs = 9, 100, 32
    g = ow.num_groups(k, gs)
    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    s = (rng.random((n, g)) * 0.018 + 0.002).astype(np.float16).astype(np.float32)
    z = rng.integers(0, 16, size=(n, g), dtype=np.uint8)
    gi = np.arange(k) // gs
    # (q - z) * s is exact in float64; rounding it to float32 is the correctly rounded fp32 product
    exact = ((q.astype(np.float64) - z[:, gi]) * s[:, gi].astype(np.float64)).astype(np.float32)
    assert np.array_equal(ow.dequantize_parts(q, s, z, gs), exact)
    # symmetric: zero-point 8
    sym = ((q.astype(np.float64) - 8) * s[:, gi]).astype(np.float32)
    assert np.array_equal(ow.dequantize_parts(q, s, None, gs), sym)
    # padded columns dequantise to exactly 0
    p = ow.pack_w4(q, s, z, gs)
    full = ow.unpack_nibbles_int32(p["qweight"]).reshape(n, -1)
    pad = full[:, k:]
    assert np.array_equal(pad, np.repeat(z[:, -1:], pad.shape[1], axis=1))
    # per-channel (group -1): one group
    s1 = rng.random((n, 1), dtype=np.float32)
    assert np.array_equal(ow.dequantize_parts(q, s1, None, -1), ((q.astype(np.float64) - 8) * s1).astype(np.float32))


@pytest.mark.parametrize("m", [0, 1, 3, 16, 33])
@pytest.mark.parametrize("n,k,gs", [(7, 100, 32), (64, 65, 16), (130, 257, 64), (5, 24, -1)])
def test_w4a16_ref_equals_float64_dequant_then_matmul(m, n, k, gs):
    """Reference test tests/test_kernels_gemm_refs.py:54-70: M=0, odd N, K not a multiple of the group."""
    rng = np.random.default_rng(n + k)
    g = ow.num_groups(k, gs)
    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    s = rng.random((n, g), dtype=np.float32) + 0.1
    z = rng.integers(0, 16, size=(n, g), dtype=np.uint8)
    x = rnd(m, k, seed=3)
    bias = rnd(n, seed=4)
    y = og.w4a16_gemm_ref(x, ow.pack_w4(q, s, z, gs), bias)
    gi = np.arange(k) // (k if gs <= 0 else gs)
    wd = (q.astype(np.float64) - z[:, gi]) * s[:, gi]
    expect = x.astype(np.float64) @ wd.T + bias
    assert y.shape == (m, n) and y.dtype == np.float32
    np.testing.assert_allclose(y, expect, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("m", [0, 1, 5, 33])
@pytest.mark.parametrize("n,k,gs", [(7, 100, 32), (64, 65, -1), (130, 256, 128)])
def test_w8a16_ref_equals_float64_brute_force(m, n, k, gs):
    """W8A16 oracle (forge/kernels/ref/gemm_w4a16.py:45-52): element-by-element q * s (exact in fp32: an int8 times an
    fp16-representable scale has at most 19 significant bits) against float64, and the packed scale transpose."""
    rng = np.random.default_rng(n * k)
    g = -(-k // (k if gs <= 0 else gs))
    q = rng.integers(-128, 128, size=(n, k), dtype=np.int64).astype(np.int8)
    s = (rng.random((n, g)) * 0.02 + 0.001).astype(np.float16).astype(np.float32)
    p = og.pack_w8(q, s, gs)
    assert p["scales"].shape == (g, n) and np.array_equal(p["scales"], s.T) and np.array_equal(p["qweight"], q)
    gsz = k if gs <= 0 else gs
    w = og.dequantize_w8(p)
    for (r, c) in [(0, 0), (n - 1, k - 1), (n // 2, k // 3), (1, gsz - 1 if gsz < k else k - 1)]:
        assert w[r, c] == np.float32(np.float64(q[r, c]) * np.float64(s[r, c // gsz]))
    x = rnd(m, k, seed=5)
    bias = rnd(n, seed=6)
    y = og.w8a16_gemm_ref(x, p, bias)
    expect = x.astype(np.float64) @ (q.astype(np.float64) * s[:, np.arange(k) // gsz]).T + bias
    assert y.shape == (m, n) and y.dtype == np.float32
    np.testing.assert_allclose(y, expect, rtol=1e-5, atol=1e-4)


def test_w4a16_ref_g_idx_act_order_and_column_sort():
    rng = np.random.default_rng(5)
    n, k, gs = 16, 64, 16
    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    s = rng.random((n, 4), dtype=np.float32) + 0.1
    g_idx = rng.permutation(np.arange(k) // gs).astype(np.int32)  # regular groups in act order
    p = ow.pack_w4(q, s, None, gs, g_idx)
    wd = (q.astype(np.float64) - 8) * s[:, g_idx]
    x = rnd(3, k)
    np.testing.assert_allclose(og.w4a16_gemm_ref(x, p), x @ wd.T, atol=1e-4)
    sp, perm = ow.sort_columns_by_group(p)
    assert sp["g_idx"] is None and sorted(perm.tolist()) == list(range(k))
    np.testing.assert_allclose(og.w4a16_gemm_ref(x[:, perm], sp), x @ wd.T, atol=1e-4)
    irregular = g_idx.copy()
    irregular[0] = (irregular[0] + 1) % 4
    assert ow.sort_columns_by_group(ow.pack_w4(q, s, None, gs, irregular)) is None


# ------------------------------------------------------------------------------------------- codecs vs torch
def test_bf16_codec_matches_torch_cast():
    rng = np.random.default_rng(6)
    vals = np.concatenate([rng.standard_normal(200000).astype(np.float32) * 10 ** rng.uniform(-30, 30, 200000).astype(np.float32),
                           np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.4e38, 1e-40, 1.00390625, 1.01171875], np.float32)])
    vals = vals.astype(np.float32)
    mine = og.f32_to_bf16(vals)
    theirs = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mine, theirs)
    assert np.array_equal(og.bf16_to_f32(theirs), torch.from_numpy(theirs.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_e4m3_decode_all_codes_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    mine = og.e4m3_decode(codes)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(mine), np.isnan(theirs))
    ok = ~np.isnan(theirs)
    assert np.array_equal(mine[ok], theirs[ok])
    assert mine[0x7E] == 448.0 and mine[0x01] == 2.0 ** -9 and np.isnan(mine[0x7F]) and np.isnan(mine[0xFF])


def test_e4m3_encode_matches_torch_cast_on_dense_sweep():
    rng = np.random.default_rng(7)
    codes = np.arange(256, dtype=np.uint8)
    grid = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    grid = grid[np.isfinite(grid)]
    mids = (np.sort(np.unique(grid))[1:] + np.sort(np.unique(grid))[:-1]) / 2  # exact ties
    vals = np.concatenate([np.linspace(-448, 448, 400001), rng.uniform(-2 ** -5, 2 ** -5, 100000), grid, mids,
                           np.nextafter(mids, np.inf), np.nextafter(mids, -np.inf), [0.0, -0.0]]).astype(np.float32)
    vals = np.clip(vals, -448, 448).astype(np.float32)
    mine = og.e4m3_encode(vals)
    theirs = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(mine, theirs)
    nan = np.array([np.nan], np.float32)
    assert og.e4m3_encode(nan)[0] == torch.from_numpy(nan).to(torch.float8_e4m3fn).view(torch.uint8).item()


# ------------------------------------------------------------------------------------------- FP8 quantiser / GEMM
@pytest.mark.parametrize("gran", ["per_tensor", "per_token", "block"])
@pytest.mark.parametrize("k", [64, 100, 300])
def test_fp8_quant_dequant_error_bound(gran, k):
    """tests/test_kernels_gemm_refs.py:134-145: |dq - x| <= |x| 2^-4 + s_max 2^-9; |q| <= 448."""
    x = rnd(7, k, scale=3.0)
    q, s = og.quantize_fp8_ref(x, gran, block=128)
    d = og.dequantize_fp8_ref(q, s, block=128)
    assert (np.abs(d - x) <= np.abs(x) * 2 ** -4 + s.max() * 2 ** -9 + 1e-6).all()
    assert np.abs(og.e4m3_decode(q)).max() <= 448.0


def test_fp8_quant_known_answers():
    """tests/test_kernels_gemm_refs.py:147-162."""
    x = rnd(4, 130)
    x[1] = 0
    q, s = og.quantize_fp8_ref(x, "per_token")
    assert s.shape == (4,) and s[1] == 1.0 and (og.e4m3_decode(q[1]) == 0).all()
    _, sb = og.quantize_fp8_ref(x, "block", block=128)
    assert sb.shape == (4, 2)
    _, s2 = og.quantize_fp8_ref(rnd(130, 70), "block2d", block=128)
    assert s2.shape == (2, 1)
    q, _ = og.quantize_fp8_ref(np.array([[1000.0, -1000.0, 1.0]], np.float32), "per_tensor", scale=np.array([1.0]))
    assert og.e4m3_decode(q).tolist() == [[448.0, -448.0, 1.0]]
    q, s = og.quantize_fp8_ref(np.array([[2.0, -4.0]], np.float32), "per_token")
    assert np.abs(og.e4m3_decode(q)).max() == 448.0 and s[0] == np.float32(4.0) / np.float32(448.0)


def test_fp8_quant_codes_match_torch_restatement():
    """Codes equal torch's own clamp + cast of x / s (an independent implementation of the same formula)."""
    x = rnd(33, 300, seed=9, scale=5.0)
    x[3, :] = 0
    for gran in ("per_token", "per_tensor", "block", "block2d"):
        q, s = og.quantize_fp8_ref(x, gran, block=64)
        sb = og.expand_scale(s, 33, 300, 64)
        t = (torch.from_numpy(x) / torch.from_numpy(np.ascontiguousarray(sb))).clamp(-448, 448).to(torch.float8_e4m3fn)
        assert np.array_equal(q, t.view(torch.uint8).numpy()), gran


@pytest.mark.parametrize("gx,gw", [("per_tensor", "per_tensor"), ("per_token", "per_channel"), ("block", "block2d")])
@pytest.mark.parametrize("m,n,k", [(1, 16, 64), (5, 40, 200), (130, 130, 260), (0, 8, 32)])
def test_fp8_gemm_ref_matches_float64_dequant(gx, gw, m, n, k):
    x, w = rnd(m, k, seed=1), rnd(n, k, seed=2)
    xq, sx = og.quantize_fp8_ref(x, gx)
    wq, sw = og.quantize_fp8_ref(w, gw)
    b = np.arange(n, dtype=np.float32)
    y = og.fp8_gemm_ref(xq, sx, wq, sw, b)
    xd = og.e4m3_decode(xq).astype(np.float64) * og.expand_scale(sx, m, k)
    wd = og.e4m3_decode(wq).astype(np.float64) * og.expand_scale(sw, n, k)
    np.testing.assert_allclose(y, xd @ wd.T + b, atol=1e-4, rtol=1e-5)
    if m:
        assert np.abs(y - (x @ w.T + b)).max() <= 0.12 * np.abs(x @ w.T).max() + 1e-3


# ------------------------------------------------------------------------------------------- INT8
# ------------------------------------------------------------------------------------------- fused RMSNorm -> fp8
def _rms64(x, w, eps):
    """``y = x / sqrt(mean(x^2) + eps) * w`` in float64 (the definition, forge/kernels/ref/gemm_fp8.py:130-150)."""
    x64 = np.asarray(x, dtype=np.float64)
    y = x64 / np.sqrt((x64 * x64).mean(axis=-1, keepdims=True) + eps)
    return y if w is None else y * np.asarray(w, dtype=np.float64)


def _rmsnorm_pin_failures(fn) -> list[str]:
    """Every check that ``fn`` (an rmsnorm_act_quant_fp8_ref candidate) fails; [] for a correct one."""
    bad = []
    # closed form on random rows (float32 arithmetic: a few ulps of pairwise-sum and sqrt error)
    for k, seed in ((1, 1), (7, 2), (64, 3), (1000, 4), (4096, 5)):
        x = rnd(5, k, seed=seed, scale=3.0).astype(np.float32)
        w = (np.abs(rnd(k, seed=seed + 10)) + 0.5).astype(np.float32)
        q, s, y = fn(x, w, 1e-6)
        y64 = _rms64(x, w, 1e-6)
        if not np.all(np.abs(y - y64) <= 2e-6 * np.abs(y64) + 1e-30):
            bad.append(f"closed form k={k}")
        q2, s2 = og.quantize_fp8_ref(y, "per_token")
        if not (np.array_equal(q, q2) and np.array_equal(s, s2)):
            bad.append(f"quantisation of y k={k}")
    # constant row c: y = c / sqrt(c^2 + eps); eps inside the root, a mean (not a sum) over K
    x = np.full((1, 16), 2.0, np.float32)
    _, _, y = fn(x, None, 0.25)
    if not np.allclose(y, 2.0 / np.sqrt(4.25), rtol=1e-7, atol=0):
        bad.append("constant row")
    # the weight multiplies after the normalisation, element by element
    _, s, y = fn(np.array([[3.0, 4.0]], np.float32), np.array([2.0, 0.5], np.float32), 1.0)
    if not np.allclose(y, np.array([[6.0, 2.0]]) / np.sqrt(13.5), rtol=1e-7, atol=0):
        bad.append("weight / eps placement")
    if not np.isclose(s[0], 6.0 / np.sqrt(13.5) / 448.0, rtol=1e-7):
        bad.append("scale = amax(y) / 448")
    # a zero row normalises to zero: scale 1, codes 0
    q, s, y = fn(np.zeros((2, 8), np.float32), np.ones(8, np.float32), 1e-6)
    if not (np.all(y == 0) and np.all(s == 1.0) and np.all(q == 0)):
        bad.append("zero row")
    return bad


def test_rmsnorm_act_quant_fp8_ref_pinned():
    assert _rmsnorm_pin_failures(og.rmsnorm_act_quant_fp8_ref) == []


def test_rmsnorm_pins_catch_planted_mistakes():
    """eps outside the root, a sum over K instead of the mean, and the weight applied before the norm all fail."""
    def eps_outside(x, w, eps):
        xf = np.asarray(x, np.float32)
        y = (xf / (np.sqrt((xf * xf).mean(-1, keepdims=True)) + np.float32(eps))).astype(np.float32)
        y = y if w is None else (y * w).astype(np.float32)
        return (*og.quantize_fp8_ref(y, "per_token"), y)

    def sum_not_mean(x, w, eps):
        xf = np.asarray(x, np.float32)
        y = (xf / np.sqrt((xf * xf).sum(-1, keepdims=True) + np.float32(eps))).astype(np.float32)
        y = y if w is None else (y * w).astype(np.float32)
        return (*og.quantize_fp8_ref(y, "per_token"), y)

    def weight_first(x, w, eps):
        xf = np.asarray(x, np.float32) * (1 if w is None else w)
        y = (xf / np.sqrt((xf * xf).mean(-1, keepdims=True) + np.float32(eps))).astype(np.float32)
        return (*og.quantize_fp8_ref(y, "per_token"), y)

    for fn in (eps_outside, sum_not_mean, weight_first):
        assert _rmsnorm_pin_failures(fn), fn.__name__


def test_int8_quant_known_answers_and_ieee_scale():
    """tests/test_kernels_gemm_refs.py:205-213 and :351-359."""
    x = rnd(9, 70, scale=2)
    q, s = og.quantize_int8_ref(x)
    assert q.dtype == np.int8 and q.min() >= -127 and (np.abs(q.astype(int)).max(axis=1) == 127).all()
    q2, _ = og.quantize_int8_ref(np.array([[0.5, 1.5, 2.5, -0.5, -1.5, 127.0]], np.float32), scale=np.array([1.0]))
    assert q2.tolist() == [[0, 2, 2, 0, -2, 127]]
    q3, _ = og.quantize_int8_ref(np.array([[300.0, -300.0]], np.float32), scale=np.array([1.0]))
    assert q3.tolist() == [[127, -127]]
    g = torch.Generator().manual_seed(0)
    xx = (torch.randn(512, 64, generator=g) * torch.rand(512, 1, generator=g) * 10).numpy()
    _, s = og.quantize_int8_ref(xx)
    assert np.array_equal(s, (np.abs(xx).max(axis=1).astype(np.float64) / 127.0).astype(np.float32))
    # zero row -> scale 1, codes 0
    q0, s0 = og.quantize_int8_ref(np.zeros((1, 5), np.float32))
    assert s0[0] == 1.0 and (q0 == 0).all()


def test_int8_quant_matches_torch_restatement():
    x = rnd(64, 257, seed=11, scale=3)
    q, s = og.quantize_int8_ref(x)
    t = torch.from_numpy(x)
    amax = t.abs().amax(dim=-1)
    ts = torch.where(amax > 0, amax / torch.full_like(amax, 127.0), torch.ones_like(amax))
    tq = torch.round(t / ts[:, None]).clamp(-127, 127).to(torch.int8)
    assert np.array_equal(s, ts.numpy()) and np.array_equal(q, tq.numpy())


def test_int8_matmul_exact_vs_int64_brute_force():
    rng = np.random.default_rng(3)
    a = rng.integers(-127, 128, size=(13, 333), dtype=np.int8)
    b = rng.integers(-127, 128, size=(11, 333), dtype=np.int8)
    brute = np.array([[sum(int(a[i, t]) * int(b[j, t]) for t in range(333)) for j in range(11)] for i in range(13)])
    assert np.array_equal(og.int8_matmul_exact(a, b), brute.astype(np.int32))
    big = og.int8_matmul_exact(np.full((1, 40000), 127, np.int8), np.full((1, 40000), 127, np.int8))
    assert int(big[0, 0]) == 127 * 127 * 40000


def test_int8_gemm_ref_epilogue_matches_torch_float32_ops():
    rng = np.random.default_rng(4)
    xq = rng.integers(-127, 128, size=(9, 70), dtype=np.int8)
    wq = rng.integers(-127, 128, size=(11, 70), dtype=np.int8)
    sx = (rng.random(9) + 0.1).astype(np.float32)
    sw = (rng.random(11) + 0.1).astype(np.float32)
    b = rng.standard_normal(11).astype(np.float32)
    y = og.int8_gemm_ref(xq, sx, wq, sw, b)
    acc = torch.from_numpy(xq.astype(np.int64) @ wq.astype(np.int64).T).float()
    ty = acc * torch.from_numpy(sx)[:, None] * torch.from_numpy(sw)[None, :] + torch.from_numpy(b)
    assert np.array_equal(y, ty.numpy())


# ------------------------------------------------------------------------------------------- compare()
def test_compare_rules():
    """tests/test_kernels_gemm_refs.py:112-130."""
    ref = rnd(8, 64)
    assert og.compare(ref + 1e-5, ref)["ok"]
    assert not og.compare(ref * 1.1, ref)["ok"]
    bad = ref.copy()
    bad[3, 3] += 0.5
    assert not og.compare(bad, ref)["ok"]
    bf = og.bf16_to_f32(og.f32_to_bf16(ref))
    assert og.compare(bf, ref, out_dtype="bfloat16")["ok"]
    nan = ref.copy()
    nan[0, 0] = np.nan
    assert not og.compare(nan, ref)["ok"] and og.compare(nan, nan)["ok"]
    inf = ref.copy()
    inf[1, 1] = np.inf
    assert og.compare(inf, inf)["ok"] and not og.compare(inf, ref)["ok"]
    assert not og.compare(ref[:4], ref)["ok"]
    ints = np.arange(10, dtype=np.int32)
    assert og.compare(ints, ints.copy(), exact=True)["ok"] and not og.compare(ints + 1, ints, exact=True)["ok"]


# ------------------------------------------------------------------------------------------- C oracle cross-check
def test_c_oracle_agrees_with_numpy_oracle():
    rng = np.random.default_rng(8)
    n, k, gs = 37, 200, 40
    g = ow.num_groups(k, gs)
    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    s = (rng.random((n, g)) * 0.02 + 0.002).astype(np.float16).astype(np.float32)
    z = rng.integers(6, 10, size=(n, g), dtype=np.uint8)
    p = ow.pack_w4(q, s, z, gs)
    assert np.array_equal(c_oracle.w4_dequant(p), ow.dequantize_parts(q, s, z, gs))
    gi = rng.permutation(np.arange(k) // gs).astype(np.int32)
    pg = ow.pack_w4(q, s, None, gs, gi)
    assert np.array_equal(c_oracle.w4_dequant(pg), ow.dequantize_parts(q, s, None, gs, gi))
    x = rnd(3, k)
    b = rnd(n, seed=2)
    np.testing.assert_allclose(c_oracle.w4a16_gemm(x, p, b), og.w4a16_gemm_ref(x, p, b), rtol=1e-5, atol=1e-5)
    a8 = rng.integers(-127, 128, size=(7, 999), dtype=np.int8)
    b8 = rng.integers(-127, 128, size=(5, 999), dtype=np.int8)
    assert np.array_equal(c_oracle.int8_gemm_i32(a8, b8), og.int8_matmul_exact(a8, b8))


def test_a_planted_oracle_mistake_is_caught():
    """Sanity of the pins: a dequantisation with the nibble order reversed inside each word must disagree."""
    rng = np.random.default_rng(10)
    q = rng.integers(0, 16, size=(4, 16), dtype=np.uint8)
    p = ow.pack_w4(q, np.ones((4, 1), np.float32), None, -1)
    words = p["qweight"].astype(np.int64) & 0xFFFFFFFF
    wrong = np.stack([(words >> (4 * (7 - j))) & 0xF for j in range(8)], axis=-1).reshape(4, 16)
    assert not np.array_equal(wrong, q) and np.array_equal(ow.unpack_w4(p)[0], q)


# ------------------------------------------------------------------------------------------- torch-CPU restatement
def test_torch_restatement_matches_numpy_oracle():
    """oracle/torch_ref.py (the CPU baseline's arithmetic) against the pinned numpy oracle."""
    from oracle import torch_ref as tr

    rng = np.random.default_rng(21)
    for n, k, gs, sym in ((40, 256, 128, False), (17, 200, 64, True), (8, 96, -1, False)):
        q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
        g = ow.num_groups(k, gs)
        s = (rng.random((n, g)) * 0.018 + 0.002).astype(np.float16).astype(np.float32)
        z = None if sym else rng.integers(0, 16, size=(n, g), dtype=np.uint8)
        p = ow.pack_w4(q, s, z, gs)
        qw, sc = torch.from_numpy(p["qweight"]), torch.from_numpy(p["scales"])
        zz = None if z is None else torch.from_numpy(p["zeros"])
        w = tr.dequantize(qw, sc, zz, k, gs).numpy()
        assert np.array_equal(w, ow.dequantize_parts(q, s, z, gs))
        x = rnd(5, k, seed=n)
        np.testing.assert_allclose(tr.w4a16_gemm(torch.from_numpy(x), qw, sc, zz, gs).numpy(), og.w4a16_gemm_ref(x, p),
                                   rtol=2e-5, atol=2e-5)
    xq, sx = og.quantize_int8_ref(rnd(9, 300, seed=3))
    wq, sw = og.quantize_int8_ref(rnd(33, 300, seed=4, scale=0.05), "per_channel")
    y = tr.int8_gemm(torch.from_numpy(xq), torch.from_numpy(sx), torch.from_numpy(wq), torch.from_numpy(sw))
    assert np.array_equal(y.numpy(), og.int8_gemm_ref(xq, sx, wq, sw))
    fq, fsx = og.quantize_fp8_ref(rnd(9, 300, seed=5))
    fw, fsw = og.quantize_fp8_ref(rnd(33, 300, seed=6, scale=0.05), "per_channel")
    y = tr.fp8_gemm(torch.from_numpy(fq).view(torch.float8_e4m3fn), torch.from_numpy(fsx),
                    torch.from_numpy(fw).view(torch.float8_e4m3fn), torch.from_numpy(fsw))
    np.testing.assert_allclose(y.numpy(), og.fp8_gemm_ref(fq, fsx, fw, fsw), rtol=2e-5, atol=1e-6)
