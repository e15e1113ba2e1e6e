"""Packed-linear modules built from a dense CPU ``nn.Linear`` (a checkpoint quantised on the host before it is moved
to the GPU), for every kind: the reference's own flow (``tests/test_kernels_gemm_ops.py:151-172``, builders at
``forge/kernels/ops_gemm.py:391-393,890-961``).

Checked here, on the CPU: the FP8 / INT8 weight codes and scales bit-exact against the oracle quantisers
(``oracle.gemm.quantize_fp8_ref`` / ``quantize_int8_ref``, restating ``forge/kernels/ref/gemm_fp8.py:43-85`` and
``gemm_int8.py:17-35``) over ragged shapes, ties, all-zero rows and blocks, saturation and NaN; the module's
dequantised weight against the dense weight (the reference test's tolerances); and the state-dict round trip into a
module made by shape.  The GPU forward of these modules is in ``tests/test_gpu_modules.py``.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from forge_amd import layouts as L
from forge_amd import ops_gemm as ops
from oracle import gemm as og
from oracle import w4 as ow


def _rnd(*shape, seed=0, scale=1.0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale


def _awkward_weight(n: int, k: int, seed: int) -> torch.Tensor:
    w = _rnd(n, k, seed=seed, scale=0.2)
    w[1] = 0.0                               # an all-zero channel: scale 1, codes 0
    w[2, : k // 2] = 1e4                     # one huge half-row
    w[3] = torch.arange(k) * 0.5 - k / 4     # exact multiples of a power of two (ties after scaling)
    return w


@pytest.mark.parametrize("n,k", [(40, 96), (33, 130), (128, 256)])
def test_int8_weight_quantiser_matches_oracle(n, k):
    w = _awkward_weight(n, k, n + k)
    q, s = L.quantize_int8_weight(w)
    qr, sr = og.quantize_int8_ref(w.numpy(), "per_channel")
    assert q.dtype == torch.int8 and s.dtype == torch.float32 and s.shape == (n,)
    assert np.array_equal(q.numpy(), qr) and np.array_equal(s.numpy(), sr.reshape(-1))


@pytest.mark.parametrize("gran,block", [("per_channel", 128), ("per_tensor", 128), ("block2d", 32), ("block2d", 128)])
@pytest.mark.parametrize("n,k", [(40, 96), (33, 130), (128, 256)])
def test_fp8_weight_quantiser_matches_oracle(gran, block, n, k):
    w = _awkward_weight(n, k, 3 * n + k)
    q, s = ops.quantize_weight_fp8(w, gran, block)
    qr, sr = og.quantize_fp8_ref(w.numpy(), gran, block=block)
    assert q.dtype == torch.float8_e4m3fn and not q.is_cuda
    assert np.array_equal(q.view(torch.uint8).numpy(), qr)
    assert np.array_equal(s.numpy(), np.asarray(sr, dtype=np.float32).reshape(s.shape))


@pytest.mark.filterwarnings("ignore:invalid value encountered in cast")  # the oracle's NaN -> int8 cast (code 0)
def test_w8a8_weight_quantisers_nan_and_saturation():
    w = torch.tensor([[1.0, -2.0, float("nan"), 0.5], [300.0, -300.0, 1.0, 0.0], [0.0, 0.0, 0.0, 0.0]])
    q8, s8 = L.quantize_int8_weight(w)
    qr, sr = og.quantize_int8_ref(w.numpy(), "per_channel")
    assert np.array_equal(q8.numpy(), qr) and np.array_equal(s8.numpy(), sr.reshape(-1))
    assert s8[0] == 1.0 and s8[2] == 1.0 and q8[1, 0] == 127 and q8[1, 1] == -127
    qf, sf = L.quantize_fp8_weight(w, "per_channel")
    qfr, sfr = og.quantize_fp8_ref(w.numpy(), "per_channel")
    assert np.array_equal(qf.view(torch.uint8).numpy(), qfr) and np.array_equal(sf.numpy(), sfr.reshape(-1))
    # a static-free amax maps to 448 exactly; an all-zero row quantises to code 0 with scale 1
    assert float(qf[1, 0].float()) == 448.0 and float(sf[2]) == 1.0 and int(qf[2].view(torch.uint8).sum()) == 0


def _dequantised(m) -> torch.Tensor:
    """The module's stored weight as a dense fp32 ``[N, K]``: the oracle's dequantisation for the weight-only kinds
    (whose ``dequantize`` runs on the GPU here), the module's own host ``dequantize`` for FP8 / INT8."""
    if m.kind == "w4a16":
        q, s, z = L.unpack_w4(m.packed())
        return torch.from_numpy(ow.dequantize_parts(q.numpy(), s.float().numpy(), None if z is None else z.numpy(),
                                                    m.group_size))
    if m.kind == "w8a16":
        return torch.from_numpy(og.dequantize_w8(og.pack_w8(m.qweight.numpy(), m.scales.float().t().numpy(),
                                                            m.group_size)))
    return m.dequantize()


# kinds and tolerances of the reference's module test (relative Frobenius error of y against the dense linear)
KINDS = [("w4a16", {"group_size": 32}, 0.25), ("w4a16", {"group_size": 32, "sym": False}, 0.2),
         ("w8a16", {}, 0.02), ("w8a16", {"group_size": 32}, 0.02), ("fp8", {}, 0.1),
         ("fp8", {"granularity": "block2d", "block": 32}, 0.1), ("fp8", {"granularity": "per_tensor"}, 0.1),
         ("int8", {}, 0.03)]


@pytest.mark.parametrize("kind,kw,tol", KINDS)
def test_make_packed_linear_from_cpu_dense_and_state_dict_roundtrip(kind, kw, tol):
    lin = nn.Linear(96, 40, bias=True)
    with torch.no_grad():
        lin.weight.copy_(_rnd(40, 96, seed=5, scale=0.2))
        lin.bias.copy_(_rnd(40, seed=6))
    m = ops.make_packed_linear(kind, lin, **kw)
    assert m.in_features == 96 and m.out_features == 40
    assert all(not t.is_cuda for t in m.state_dict().values())
    # the stored weight, dequantised, reproduces the dense one within the reference's tolerance for this kind
    x = _rnd(3, 96, seed=7)
    dense = _dequantised(m)
    with torch.no_grad():
        y = nn.functional.linear(x, dense, m.bias)
        ref = nn.functional.linear(x, lin.weight, lin.bias)
    assert dense.shape == (40, 96) and float((y - ref).norm() / ref.norm()) < tol
    assert "bias" in m.state_dict() and torch.equal(m.bias.detach(), lin.bias.detach())
    # the artifact-loading route: an empty module of the same shape takes the state dict bit for bit
    fresh = ops.make_packed_linear(kind, in_features=96, out_features=40, bias=lin.bias, **kw)
    fresh.load_state_dict(m.state_dict())
    for name, t in m.state_dict().items():
        got = fresh.state_dict()[name]
        assert got.dtype == t.dtype and torch.equal(got.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else got,
                                                    t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t), name


def test_fp8_and_int8_modules_from_cpu_codes_match_oracle():
    lin = nn.Linear(130, 33, bias=False)
    with torch.no_grad():
        lin.weight.copy_(_awkward_weight(33, 130, 11))
    w = lin.weight.detach().numpy()
    m8 = ops.make_packed_linear("int8", lin)
    qr, sr = og.quantize_int8_ref(w, "per_channel")
    assert np.array_equal(m8.weight_int8.numpy(), qr) and np.array_equal(m8.weight_scale.numpy(), sr.reshape(-1))
    mf = ops.make_packed_linear("fp8", lin, granularity="block2d", block=32)
    qf, sf = og.quantize_fp8_ref(w, "block2d", block=32)
    assert np.array_equal(mf.weight_fp8.view(torch.uint8).numpy(), qf)
    assert np.array_equal(mf.weight_scale.numpy(), np.asarray(sf, dtype=np.float32).reshape(mf.weight_scale.shape))
