"""Oracle restatement of the GEMM-family reference oracles (numpy, CPU) -- test infrastructure only.

Reference files:
* ``forge/kernels/ref/gemm_w4a16.py:9-27``  -- W4A16: dequantise to fp32, ``x.float() @ W.T (+ bias.float())``
* ``forge/kernels/ref/gemm_w4a16.py:45-52`` -- W8A16: ``q * s`` in fp32, then the same GEMM
* ``forge/kernels/ref/gemm_fp8.py:22-127`` -- FP8 e4m3fn quantiser (per-tensor / per-token / 1xB / BxB), dequant, GEMM
* ``forge/kernels/ref/gemm_int8.py:8-85``  -- INT8 per-token/channel quantiser, exact int32 GEMM, fp32 epilogue
* ``forge/kernels/ref/gemm_common.py:27-80`` -- ``compare`` tolerance rule

Number formats without a numpy dtype are carried as bit patterns: bf16 as ``uint16``, e4m3fn as ``uint8``.  The
codecs below are written from the format definitions (bf16 = top half of an IEEE binary32, round-half-even;
OCP E4M3 "FN": bias 7, 3 mantissa bits, no infinities, NaN = S.1111.111, max 448).

Pinning (``tests/test_oracle_pinned.py``): the codecs are checked exhaustively / on dense sweeps against torch's
own casts (an independent library implementation); the quantisers against the reference tests' known answers
(``tests/test_kernels_gemm_refs.py:147-162,205-222,351-359``); the GEMMs against float64 / int64 brute force.
"""
from __future__ import annotations

import numpy as np

from .w4 import dequantize_parts, unpack_w4

FP8_MAX = 448.0


# ---------------------------------------------------------------------------------------------------- codecs
def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(u16).astype(np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round-half-even; NaN stays NaN (quiet bit forced)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & np.uint64(0x7FFFFFFF)) > np.uint64(0x7F800000)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    r = np.where(nan, (u >> np.uint64(16)) | np.uint64(0x40), r)
    return (r & np.uint64(0xFFFF)).astype(np.uint16)


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """OCP e4m3fn code -> float32: ``e = (c>>3)&15, m = c&7``; subnormal ``m*2^-9``, normal ``(8+m)*2^(e-10)``."""
    c = np.asarray(codes).astype(np.uint8).astype(np.int64)
    e = (c >> 3) & 0xF
    m = c & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.exp2(e.astype(np.float64) - 10.0))
    mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
    return np.where(c & 0x80, -mag, mag).astype(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 (already clamped to +-448) -> e4m3fn code, round-half-even on the 3-bit mantissa.

    Subnormal range ``|x| < 2^-6``: code = rint(|x| * 2^9) (0..8; 8 is the smallest normal, also correct).
    Normal range: keep the binary32 exponent, round the 23-bit mantissa to 3 bits (carry bumps the exponent).
    NaN -> 0x7F (sign kept), like torch's cast.
    """
    xf = np.asarray(x, dtype=np.float32)
    sign = (xf.view(np.uint32) >> np.uint32(31)).astype(np.uint8) << np.uint8(7)
    a = np.abs(xf).astype(np.float32)
    nan = np.isnan(a)
    a = np.where(nan, np.float32(0), a)
    sub_code = np.rint(a.astype(np.float64) * 512.0).astype(np.int64)
    bits = a.view(np.uint32).astype(np.int64)
    e = (bits >> 23) - 127
    mant = bits & 0x7FFFFF
    lsb = (mant >> 20) & 1
    mr = mant + 0x7FFFF + lsb
    carry = mr >> 23
    m3 = np.where(carry == 1, 0, mr >> 20)
    e2 = e + carry
    norm_code = ((e2 + 7) << 3) | m3
    code = np.where(a < 2.0 ** -6, sub_code, norm_code).astype(np.int64)
    code = np.where(nan, 0x7F, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


# ---------------------------------------------------------------------------------------------------- W4A16
def w4a16_gemm_ref(x: np.ndarray, packed: dict, bias: np.ndarray | None = None) -> np.ndarray:
    """``Y = X @ dequant(W)^T + bias`` in fp32 (``forge/kernels/ref/gemm_w4a16.py:9-27``).

    ``x`` float32 ``[M,K]`` (bf16/fp16 inputs widened exactly), ``packed`` from :func:`oracle.w4.pack_w4` with float32
    scales or float16 scales (widened here).  Returns float32 ``[M,N]``; the caller casts to the output dtype.
    """
    q, s, z = unpack_w4(packed)
    w = dequantize_parts(q, s.astype(np.float32), z, packed["group_size"], packed["g_idx"])
    y = np.asarray(x, dtype=np.float32) @ w.T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)
    return y.astype(np.float32)


# ---------------------------------------------------------------------------------------------------- W8A16
def pack_w8(q: np.ndarray, scales: np.ndarray, group_size: int = -1) -> dict:
    """Portable_row W8 (``forge/kernels/layouts/w8.py:83-94``): ``qweight int8 [N, K]`` as given, ``scales [N, G]``
    stored transposed as ``[G, N]``."""
    q = np.asarray(q, dtype=np.int8)
    n, k = q.shape
    gs = k if group_size is None or group_size <= 0 else int(group_size)
    g = -(-k // gs)
    s = np.asarray(scales)
    if s.shape != (n, g):
        raise ValueError(f"scales must be [N={n}, G={g}], got {s.shape}")
    return {"qweight": q.copy(), "scales": np.ascontiguousarray(s.T), "n": n, "k": k, "group_size": int(group_size)}


def dequantize_w8(packed: dict) -> np.ndarray:
    """``W[n, k] = q[n, k] * scales[k // gs, n]`` in float32 (``forge/kernels/layouts/w8.py:101-104``)."""
    q, s = packed["qweight"], np.asarray(packed["scales"], dtype=np.float32)
    n, k = q.shape
    gs = k if packed["group_size"] <= 0 else packed["group_size"]
    gi = np.arange(k) // gs
    return (q.astype(np.float32) * s[gi, :].T).astype(np.float32)


def w8a16_gemm_ref(x: np.ndarray, packed: dict, bias: np.ndarray | None = None) -> np.ndarray:
    """``Y = X @ dequant(Wq)^T + bias`` in fp32 (``forge/kernels/ref/gemm_w4a16.py:45-52``)."""
    y = np.asarray(x, dtype=np.float32) @ dequantize_w8(packed).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)
    return y.astype(np.float32)


# ---------------------------------------------------------------------------------------------------- FP8
def _safe_scale(amax: np.ndarray, fmax: float) -> np.ndarray:
    """``amax / fmax`` with 1.0 where ``amax > 0`` is false (zero rows, and NaN rows as torch.where gives)."""
    amax = np.asarray(amax, dtype=np.float32)
    with np.errstate(invalid="ignore"):
        return np.where(amax > 0, amax / np.float32(fmax), np.float32(1.0)).astype(np.float32)


def _nan_amax(a: np.ndarray, axis=None) -> np.ndarray:
    """max |a| that propagates NaN (torch.amax semantics)."""
    return np.max(np.abs(a), axis=axis)


def quantize_fp8_ref(x: np.ndarray, granularity: str = "per_token", *, block: int = 128,
                     scale: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """FP8 e4m3fn quantisation of ``x [M,K]`` float32 (``forge/kernels/ref/gemm_fp8.py:43-85``).

    Returns ``(codes uint8 [M,K], scale float32)``; ``q = clamp(x / s, +-448)`` cast with round-half-even.
    """
    x2 = np.asarray(x, dtype=np.float32)
    m, k = x2.shape
    g = "per_token" if granularity == "per_channel" else granularity
    if g == "per_tensor":
        amax = _nan_amax(x2).reshape(1) if x2.size else np.zeros(1, np.float32)
        s = _safe_scale(amax, FP8_MAX) if scale is None else np.asarray(scale, np.float32).reshape(1)
        sb = s.reshape(1, 1)
    elif g == "per_token":
        s = _safe_scale(_nan_amax(x2, axis=-1), FP8_MAX) if scale is None else np.asarray(scale, np.float32).reshape(m)
        sb = s.reshape(m, 1)
    elif g == "block":
        kb = -(-k // block)
        xp = np.pad(x2, ((0, 0), (0, kb * block - k)))
        amax = _nan_amax(xp.reshape(m, kb, block), axis=-1)
        s = _safe_scale(amax, FP8_MAX) if scale is None else np.asarray(scale, np.float32).reshape(m, kb)
        sb = np.repeat(s, block, axis=1)[:, :k]
    elif g == "block2d":
        nb, kb = -(-m // block), -(-k // block)
        xp = np.pad(x2, ((0, nb * block - m), (0, kb * block - k)))
        amax = _nan_amax(xp.reshape(nb, block, kb, block), axis=(1, 3))
        s = _safe_scale(amax, FP8_MAX) if scale is None else np.asarray(scale, np.float32).reshape(nb, kb)
        sb = np.repeat(np.repeat(s, block, axis=0), block, axis=1)[:m, :k]
    else:
        raise ValueError(f"unknown granularity {granularity!r}")
    with np.errstate(invalid="ignore", divide="ignore"):
        v = (x2 / sb).astype(np.float32)
    v = np.where(np.isnan(v), v, np.clip(v, -FP8_MAX, FP8_MAX)).astype(np.float32)
    return e4m3_encode(v), np.ascontiguousarray(s.astype(np.float32))


def rmsnorm_act_quant_fp8_ref(x: np.ndarray, weight: np.ndarray | None, eps: float = 1e-6, *,
                              granularity: str = "per_token", block: int = 128) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Fused producer oracle (``forge/kernels/ref/gemm_fp8.py:130-150``): ``y = x * rsqrt(mean(x^2) + eps) * w`` in fp32
    (rsqrt = 1 / sqrt, each correctly rounded), then FP8 quantisation of ``y``.  Returns ``(codes, scale, y)``."""
    xf = np.asarray(x, dtype=np.float32)
    ms = (xf * xf).mean(axis=-1, keepdims=True, dtype=np.float32)
    r = (np.float32(1.0) / np.sqrt((ms + np.float32(eps)).astype(np.float32))).astype(np.float32)
    y = (xf * r).astype(np.float32)
    if weight is not None:
        y = (y * np.asarray(weight, dtype=np.float32)).astype(np.float32)
    q, s = quantize_fp8_ref(y, granularity, block=block)
    return q, s, y


def expand_scale(scale: np.ndarray, rows: int, k: int, block: int = 128) -> np.ndarray:
    """Broadcast a scale tensor to ``[rows, k]`` (``forge/kernels/ref/gemm_fp8.py:88-101``)."""
    s = np.asarray(scale, dtype=np.float32)
    if s.size == 1:
        return np.broadcast_to(s.reshape(1, 1), (rows, k))
    if s.ndim == 1:
        if s.size != rows:
            raise ValueError(f"1-D scale has {s.size} entries, expected {rows}")
        return np.broadcast_to(s.reshape(rows, 1), (rows, k))
    if s.ndim == 2:
        if s.shape[0] == rows:
            return np.repeat(s, block, axis=1)[:, :k]
        return np.repeat(np.repeat(s, block, axis=0), block, axis=1)[:rows, :k]
    raise ValueError(f"unsupported scale shape {s.shape}")


def dequantize_fp8_ref(codes: np.ndarray, scale: np.ndarray, block: int = 128) -> np.ndarray:
    """``q.float() * expand(scale)`` (``forge/kernels/ref/gemm_fp8.py:104-107``)."""
    c = np.asarray(codes)
    return (e4m3_decode(c) * expand_scale(scale, c.shape[0], c.shape[1], block)).astype(np.float32)


def fp8_gemm_ref(xq: np.ndarray, sx: np.ndarray, wq: np.ndarray, sw: np.ndarray, bias: np.ndarray | None = None,
                 *, block: int = 128) -> np.ndarray:
    """``Y = dq(Xq) @ dq(Wq)^T + bias`` in fp32 (``forge/kernels/ref/gemm_fp8.py:110-127``)."""
    y = dequantize_fp8_ref(xq, sx, block) @ dequantize_fp8_ref(wq, sw, block).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)
    return y.astype(np.float32)


# ---------------------------------------------------------------------------------------------------- INT8
def quantize_int8_ref(x: np.ndarray, granularity: str = "per_token",
                      scale: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric int8 (``forge/kernels/ref/gemm_int8.py:8-35``): ``s = amax /_IEEE 127`` (1 where amax>0 is false),
    ``q = clamp(round_half_even(x /_IEEE s), -127, 127)``."""
    x2 = np.asarray(x, dtype=np.float32)
    if granularity in ("per_token", "per_channel"):
        amax = _nan_amax(x2, axis=-1).astype(np.float32)
        with np.errstate(invalid="ignore"):
            s = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32) if scale is None \
                else np.asarray(scale, np.float32).reshape(-1)
        sb = s.reshape(-1, 1)
    elif granularity == "per_tensor":
        amax = (_nan_amax(x2).reshape(1) if x2.size else np.zeros(1)).astype(np.float32)
        s = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32) if scale is None \
            else np.asarray(scale, np.float32).reshape(1)
        sb = s.reshape(1, 1)
    else:
        raise ValueError(f"unknown granularity {granularity!r}")
    q = np.clip(np.rint((x2 / sb).astype(np.float32)), -127, 127).astype(np.int8)
    return q, np.ascontiguousarray(s.astype(np.float32))


def int8_matmul_exact(xq: np.ndarray, wq: np.ndarray) -> np.ndarray:
    """``int32 [M,N] = xq @ wq^T`` exactly (``forge/kernels/ref/gemm_int8.py:62-65``): the products and every partial
    sum are integers below ``K * 127^2 < 2^53``, so a float64 matmul holds them exactly (checked against int64
    brute force in the oracle pins)."""
    xq, wq = np.asarray(xq), np.asarray(wq)
    assert xq.shape[-1] * 127 * 128 < 2 ** 53
    acc = xq.astype(np.float64) @ wq.astype(np.float64).T
    return np.rint(acc).astype(np.int64).astype(np.int32)


def int8_gemm_ref(xq: np.ndarray, sx: np.ndarray, wq: np.ndarray, sw: np.ndarray, bias: np.ndarray | None = None,
                  acc: np.ndarray | None = None) -> np.ndarray:
    """``Y = (acc_int32.float() * sx[:,None]) * sw[None,:] + bias`` with one fp32 rounding per operation
    (``forge/kernels/ref/gemm_int8.py:68-85``).  ``acc`` may be passed to reuse a precomputed accumulator."""
    a = int8_matmul_exact(xq, wq) if acc is None else acc
    sxa = np.asarray(sx, dtype=np.float32).reshape(-1, 1) if np.size(sx) != 1 else np.asarray(sx, np.float32).reshape(1, 1)
    swa = np.asarray(sw, dtype=np.float32).reshape(1, -1) if np.size(sw) != 1 else np.asarray(sw, np.float32).reshape(1, 1)
    y = (a.astype(np.float32) * sxa).astype(np.float32) * swa
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)
    return y.astype(np.float32)


# ---------------------------------------------------------------------------------------------------- compare
SPEC_TOL = {"rel": 2e-3, "abs": 1e-3, "rel_norm": 2e-2}  # forge/kernels/specs/{w4a16_gemm,fp8_gemm,int8_w8a8_gemm}.yaml

EPS = {"float32": float(np.finfo(np.float32).eps), "float16": float(np.finfo(np.float16).eps), "bfloat16": 2.0 ** -7}


def compare(out: np.ndarray, ref: np.ndarray, tol: dict | None = None, *, out_dtype: str = "float32",
            exact: bool = False, slack: float = 1.0) -> dict:
    """Tolerance rule of ``forge/kernels/ref/gemm_common.py:36-80``::

        max|out-ref| <= abs + max(rel, 2*eps(out_dtype)) * max|ref|   and   <= abs + rel_norm * max|ref|

    with non-finite entries required to match positionally.  ``exact`` demands bit equality.
    """
    out, ref = np.asarray(out), np.asarray(ref)
    if out.shape != ref.shape:
        return {"ok": False, "detail": f"shape {out.shape} != {ref.shape}"}
    if exact:
        eq = bool(np.array_equal(out, ref.astype(out.dtype)))
        return {"ok": eq, "detail": "bit-exact" if eq else "bit mismatch"}
    t = dict(SPEC_TOL, **(tol or {}))
    o, r = out.astype(np.float64), ref.astype(np.float64)
    fo, fr = np.isfinite(o), np.isfinite(r)
    same_nonfinite = (o == r) | (np.isnan(o) & np.isnan(r))
    nonfinite_bad = int(((fo != fr) | (~fo & ~fr & ~same_nonfinite)).sum())
    both = fo & fr
    err = float(np.abs(o[both] - r[both]).max()) if both.any() else 0.0
    ref_max = float(np.abs(r[both]).max()) if both.any() else 0.0
    eps = EPS[out_dtype]
    thr = min(t["abs"] + max(t["rel"], 2.0 * eps) * ref_max, t["abs"] + t["rel_norm"] * ref_max) * slack
    ok = nonfinite_bad == 0 and err <= thr
    return {"ok": ok, "max_abs_err": err, "ref_max": ref_max, "rel_err": err / ref_max if ref_max else 0.0,
            "thr": thr, "nonfinite_mismatch": nonfinite_bad,
            "detail": f"max_abs_err={err:.3e} thr={thr:.3e} ref_max={ref_max:.3e} nonfinite_mismatch={nonfinite_bad}"}


def max_rel_err(out: np.ndarray, ref: np.ndarray) -> float:
    """North-star parity figure: ``max|out - ref| / max|ref|`` over finite entries (bar: <= 1e-2)."""
    o, r = np.asarray(out, np.float64), np.asarray(ref, np.float64)
    both = np.isfinite(o) & np.isfinite(r)
    if not both.any():
        return 0.0
    rm = float(np.abs(r[both]).max())
    return float(np.abs(o[both] - r[both]).max()) / rm if rm else float(np.abs(o[both]).max())
