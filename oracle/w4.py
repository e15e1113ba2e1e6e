"""Oracle restatement of the portable_row W4 layout (numpy, CPU) -- test infrastructure only.

Reference: ``forge/kernels/layouts/w4.py`` (pack/unpack/dequantize, act-order sort), ``forge/kernels/layouts/bits.py``
(nibble packing) and ``forge/kernels/layouts/layout.py:124-198`` (layout id).

Storage rule (``w4.py:15-17``):

* ``qweight int32 [N, ceil(K/8)]``: nibble ``j`` (bits ``4j..4j+3``) of word ``w`` holds ``q[n, 8w + j]``;
* ``scales [G, N]``: the transpose of the logical ``[N, G]`` scales;
* ``zeros int32 [G, ceil(N/8)]``: nibble ``j`` of word ``v`` holds ``zero[8v + j, g]``;
* K padding columns carry the zero-point of the column's group, so they dequantise to exactly 0 (``w4.py:232-237``).

Pinning (``tests/test_oracle_pinned.py``): brute-force per-element pack on tiny shapes, the closed-form
``W = (q - z) * s`` in float64, the layout-id hash recomputed from the storage signature, and the reference's
property matrix (pack -> unpack identity over shapes/groups/sym, ``tests/test_kernels_gemm_layouts.py:136-151``).
"""
from __future__ import annotations

import hashlib
import json

import numpy as np


def layout_id(bits: int = 4) -> str:
    """Deterministic portable-row layout id: ``w{bits}.portable_row.v1-<blake2b-3 of the storage signature>``
    (``forge/kernels/layouts/layout.py:135-137,167-198``)."""
    sig = {
        "kind": "portable_row",
        "bits": bits,
        "atom": "",
        "tile_k": 8 if bits == 4 else 1,
        "tile_n": 1,
        "interleave": list(range(8)),
        "scales": {"orientation": "col_contig_GxN", "pad_n_to": 1},
        "swizzle": {"kind": "none"},
    }
    blob = json.dumps(sig, sort_keys=True, separators=(",", ":")).encode()
    return f"w{bits}.portable_row.v1-{hashlib.blake2b(blob, digest_size=3).hexdigest()}"


def effective_group(group_size: int, k: int) -> int:
    """``forge/kernels/layouts/w4.py:47-49``: ``-1``/``0`` means one group over the whole row."""
    return int(k) if group_size is None or group_size <= 0 else int(group_size)


def num_groups(k: int, group_size: int) -> int:
    """``forge/kernels/layouts/w4.py:52-53``."""
    return -(-int(k) // effective_group(group_size, k))


def pack_nibbles_int32(nib: np.ndarray) -> np.ndarray:
    """``nib[..., 8]`` (0..15) -> int32 with nibble ``j`` at bits ``4j`` (``forge/kernels/layouts/bits.py:24-29``)."""
    nib = np.asarray(nib)
    assert nib.shape[-1] == 8
    acc = np.zeros(nib.shape[:-1], dtype=np.uint64)
    for j in range(8):
        acc |= (nib[..., j].astype(np.uint64) & np.uint64(0xF)) << np.uint64(4 * j)
    return acc.astype(np.uint32).view(np.int32)


def unpack_nibbles_int32(words: np.ndarray) -> np.ndarray:
    """int32 ``[...]`` -> uint8 ``[..., 8]`` (``forge/kernels/layouts/bits.py:32-35``)."""
    w = np.asarray(words).astype(np.int32).view(np.uint32).astype(np.uint64)
    out = np.empty(w.shape + (8,), dtype=np.uint8)
    for j in range(8):
        out[..., j] = ((w >> np.uint64(4 * j)) & np.uint64(0xF)).astype(np.uint8)
    return out


def pack_w4(q: np.ndarray, scales: np.ndarray, zeros: np.ndarray | None = None, group_size: int = 128,
            g_idx: np.ndarray | None = None) -> dict:
    """Portable-row packer (``forge/kernels/layouts/w4.py:203-257``, portable branch only).

    ``q uint8 [N,K]`` (0..15), ``scales [N,G]`` (any float dtype, kept), ``zeros uint8 [N,G]`` or None (symmetric,
    zero-point 8, ``w4.py:229``), optional ``g_idx int32 [K]``.  Returns a dict with the stored tensors.
    """
    q = np.asarray(q)
    n, k = q.shape
    g = scales.shape[1]
    gs = effective_group(group_size, k)
    k_pad = -(-k // 8) * 8
    zp = np.asarray(zeros).astype(np.uint8) if zeros is not None else np.full((n, g), 8, dtype=np.uint8)
    qp = np.zeros((n, k_pad), dtype=np.uint8)
    qp[:, :k] = q
    if k_pad > k:
        if g_idx is None:
            gk = np.minimum(np.arange(k, k_pad) // gs, g - 1)
        else:
            gk = np.repeat(np.asarray(g_idx)[-1], k_pad - k).astype(np.int64)
        qp[:, k:] = zp[:, gk]
    qweight = pack_nibbles_int32(qp.reshape(n, k_pad // 8, 8))
    sc = np.ascontiguousarray(np.asarray(scales).T)
    zq = None
    if zeros is not None:
        n8 = -(-n // 8) * 8
        zt = np.zeros((g, n8), dtype=np.uint8)
        zt[:, :n] = zp.T
        zq = pack_nibbles_int32(zt.reshape(g, n8 // 8, 8))
    gi = None if g_idx is None else np.asarray(g_idx).astype(np.int32)
    return {"qweight": qweight, "scales": sc, "zeros": zq, "g_idx": gi, "n": n, "k": k, "group_size": int(group_size)}


def unpack_w4(p: dict) -> tuple[np.ndarray, np.ndarray, np.ndarray | None]:
    """Exact inverse of :func:`pack_w4` (``forge/kernels/layouts/w4.py:260-281``, portable branch)."""
    n, k = p["n"], p["k"]
    nib = unpack_nibbles_int32(p["qweight"])
    q = nib.reshape(nib.shape[0], -1)[:n, :k].copy()
    scales = np.ascontiguousarray(p["scales"][:, :n].T)
    zeros = None
    if p["zeros"] is not None:
        zn = unpack_nibbles_int32(p["zeros"])
        zeros = np.ascontiguousarray(zn.reshape(zn.shape[0], -1)[:, :n].T)
    return q, scales, zeros


def dequantize_parts(q: np.ndarray, scales_f32: np.ndarray, zeros: np.ndarray | None, group_size: int,
                     g_idx: np.ndarray | None = None) -> np.ndarray:
    """fp32 ``W[n,k] = (q[n,k] - z[n,g(k)]) * s[n,g(k)]`` (``forge/kernels/layouts/w4.py:294-305``).

    ``scales_f32`` are the logical ``[N,G]`` scales already widened to float32 (exact for fp16/bf16 inputs).
    The subtraction is exact; the product is one fp32 rounding, the same single rounding torch performs.
    """
    n, k = q.shape
    gi = np.arange(k) // effective_group(group_size, k) if g_idx is None else np.asarray(g_idx).astype(np.int64)
    s = np.asarray(scales_f32, dtype=np.float32)[:, gi]
    z = np.float32(8.0) if zeros is None else np.asarray(zeros).astype(np.float32)[:, gi]
    return ((q.astype(np.float32) - z) * s).astype(np.float32)


def sort_columns_by_group(p: dict) -> tuple[dict, np.ndarray] | None:
    """Act-order column sort (``forge/kernels/layouts/w4.py:308-337``): stable-sort K columns by group id so each
    group is contiguous.  Returns ``(sorted_packed, perm)`` with ``perm[j]`` = original column at position ``j``,
    or None when there is no ``g_idx`` or the group sizes are irregular."""
    if p["g_idx"] is None:
        return None
    k = p["k"]
    gs, g = effective_group(p["group_size"], k), int(p["scales"].shape[0])
    gi = np.asarray(p["g_idx"]).astype(np.int64)
    if gi.size != k or gi.min() < 0 or gi.max() >= g:
        return None
    want = np.full(g, gs, dtype=np.int64)
    want[-1] = k - gs * (g - 1)
    if want[-1] <= 0 or not np.array_equal(np.bincount(gi, minlength=g), want):
        return None
    perm = np.argsort(gi, kind="stable")
    q, s, z = unpack_w4(p)
    return pack_w4(q[:, perm], s, z, p["group_size"], None), perm.astype(np.int32)
