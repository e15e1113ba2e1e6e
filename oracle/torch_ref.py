"""torch-CPU restatement of the reference's GEMM oracles -- test and measurement infrastructure only (imported by
tests/ and by bench.py's cpu_baseline, never by the product).

The reference's oracles are torch code (``forge/kernels/ref/gemm_w4a16.py:9-27``, ``ref/gemm_fp8.py:104-127``,
``ref/gemm_int8.py:62-85``); this module states the same arithmetic with torch on the CPU so that the CPU baseline
runs the reference's algorithm on all the host threads given to it, next to the numpy oracle in ``oracle/gemm.py``
that the parity tests use.

* ``w4a16_gemm``: portable_row words -> codes (nibble ``j`` of word ``w`` is column ``8w + j``), ``W = (q - z) * s`` in
  fp32 (zero-point 8 when symmetric), then ``x.float() @ W^T``.
* ``fp8_gemm``: ``(float(xq) * sx) @ (float(wq) * sw)^T`` in fp32 (per-token x per-channel scales).
* ``int8_gemm``: the int32 accumulator through a float64 matmul (exact: every partial sum is an integer below 2^53),
  then ``(float32(acc) * sx) * sw`` with one fp32 rounding per operation.

Pinned in ``tests/test_oracle_pinned.py`` against the numpy oracle: dequantisation and the INT8 results bit for bit,
the fp32 GEMMs within fp32 summation-order tolerance.
"""
from __future__ import annotations

import torch


def unpack_codes(qweight: torch.Tensor, k: int) -> torch.Tensor:
    """``int32 [N, ceil(K/8)]`` portable_row words -> ``int32 [N, K]`` codes."""
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    q = (qweight.unsqueeze(-1) >> shifts) & 0xF
    return q.reshape(qweight.shape[0], -1)[:, :k]


def dequantize(qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor | None, k: int,
               group_size: int) -> torch.Tensor:
    """fp32 ``[N, K]`` weight ``(q - z) * s`` (``forge/kernels/layouts/w4.py:294-305``)."""
    n = qweight.shape[0]
    gs = k if group_size <= 0 else group_size
    cols = torch.arange(k) // gs
    q = unpack_codes(qweight, k).float()
    s = scales.float()[:, :n].t().index_select(1, cols)
    if zeros is None:
        z = torch.full_like(q, 8.0)
    else:
        z = unpack_codes(zeros, n).t().float().index_select(1, cols)
    return (q - z) * s


def w4a16_gemm(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor | None,
               group_size: int) -> torch.Tensor:
    """``x.float() @ dequant(W)^T`` in fp32 (``forge/kernels/ref/gemm_w4a16.py:9-27``)."""
    return x.float() @ dequantize(qweight, scales, zeros, x.shape[-1], group_size).t()


def fp8_gemm(xq: torch.Tensor, sx: torch.Tensor, wq: torch.Tensor, sw: torch.Tensor) -> torch.Tensor:
    """``dq(xq) @ dq(wq)^T`` in fp32 with per-row scales on both sides (``forge/kernels/ref/gemm_fp8.py:110-127``)."""
    return (xq.float() * sx.float().reshape(-1, 1)) @ (wq.float() * sw.float().reshape(-1, 1)).t()


def int8_gemm(xq: torch.Tensor, sx: torch.Tensor, wq: torch.Tensor, sw: torch.Tensor) -> torch.Tensor:
    """Exact int32 accumulator, then ``(acc * sx) * sw`` in fp32 (``forge/kernels/ref/gemm_int8.py:62-85``)."""
    acc = torch.round(xq.double() @ wq.double().t()).to(torch.int32)
    return (acc.float() * sx.float().reshape(-1, 1)) * sw.float().reshape(1, -1)
