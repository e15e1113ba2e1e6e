"""GPU parity of W4A16's dequantise + library GEMM route (the reference's large-M route,
forge/kernels/triton/gemm_w4_dequant.py:194-256): the weights dequantised once into the workspace by the dense
dequantisation kernel, then hipBLASLt's bf16 / fp16 GEMM with the bias in its epilogue.  The policy takes it from 768
rows; forced through config={"impl": "dequant_gemm"} (the reference's "dequant_matmul") at any M.  Cases: bf16 / fp16
x, bias in x's dtype / fp32 / none, a bias type the route does not take (the fused kernel serves the call), weights
large enough to go through in two channel chunks, act-order weights (the sorted weight's perm keeps them on the fused
kernel; forcing the route then fails), run-to-run reproducibility.

Bar: max|y - ref| / max|ref| <= 1e-2 of the fp32 oracle plus the reference's compare() rule.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from forge_amd import layouts as L
from forge_amd import ops_gemm as ops
from forge_amd.errors import ForgeError
from oracle import gemm as og
from tests._util import assert_close, gen, oracle_packed, to_f32, w4_parts, x_act

pytestmark = pytest.mark.gpu
DEV = "cuda"
ODT = {torch.bfloat16: "bfloat16", torch.float16: "float16"}


def _run(m, n, k, xdt, bdt, *, seed, config=None, sym=False):
    q, s, z = w4_parts(n, k, 128, sym, seed=seed)
    p = L.pack_w4(q, s, z, 128).to(DEV)
    x = x_act(m, k, xdt, seed=seed + 1)
    b = None if bdt is None else (torch.randn(n, generator=gen(seed + 2)) * 0.5).to(bdt)
    bd = None if b is None else b.to(DEV)
    y = ops.w4a16_linear(x.to(DEV), p, bd, config=config)
    assert ops.last_path("w4a16_linear") == "hip" and y.dtype == xdt
    ref = og.w4a16_gemm_ref(to_f32(x), oracle_packed(q, s, z, 128), None if b is None else to_f32(b))
    return y, ref, (x, p, bd)


@pytest.mark.parametrize("m,kn,xdt,bdt", [
    (768, (4096, 28672), torch.bfloat16, torch.bfloat16),
    (1024, (4096, 6144), torch.bfloat16, torch.bfloat16),
    (1500, (4096, 6144), torch.float16, torch.float32),
    (1024, (14336, 4096), torch.bfloat16, None),
    (2048, (4096, 4096), torch.float16, torch.float16),
])
def test_policy_takes_the_route_from_768_rows(m, kn, xdt, bdt):
    k, n = kn
    y, ref, (x, p, bd) = _run(m, n, k, xdt, bdt, seed=m + n)
    assert_close(y.cpu(), ref, ODT[xdt], what=f"dequant+gemm m={m} k={k} n={n}")
    assert torch.equal(y, ops.w4a16_linear(x.to(DEV), p, bd)), "not reproducible run to run"
    # the same call forced through the route gives the same bits
    assert torch.equal(y, ops.w4a16_linear(x.to(DEV), p, bd, config={"impl": "dequant_gemm"}))


@pytest.mark.parametrize("m,xdt,bdt", [(64, torch.bfloat16, torch.float32), (5, torch.float16, None),
                                       (300, torch.bfloat16, torch.bfloat16)])
def test_forced_route_at_few_rows(m, xdt, bdt):
    y, ref, _ = _run(m, 2048, 1024, xdt, bdt, seed=m, config={"impl": "dequant_matmul"}, sym=(m == 5))
    assert_close(y.cpu(), ref, ODT[xdt], what=f"forced dequant+gemm m={m}")


def test_bias_type_the_route_does_not_take_falls_back():
    """bf16 x with an fp16 bias: the fused prefill kernel serves the call (same bar)."""
    y, ref, _ = _run(1024, 4096, 4096, torch.bfloat16, torch.float16, seed=11)
    assert_close(y.cpu(), ref, "bfloat16", what="fp16 bias fallback")
    with pytest.raises(ForgeError):
        _run(64, 256, 512, torch.bfloat16, torch.float16, seed=12, config={"impl": "dequant_gemm"})


def test_two_channel_chunks():
    """33024 x 8192 weights dequantise to 541 MB, over the 512 MB chunk: two dequantise + GEMM passes."""
    y, ref, _ = _run(64, 33024, 8192, torch.bfloat16, torch.bfloat16, seed=21, config={"impl": "dequant_gemm"})
    assert_close(y.cpu(), ref, "bfloat16", what="two chunks")


def test_act_order_stays_on_the_fused_kernel():
    n, k, m = 1024, 2048, 1024
    q, s, z = w4_parts(n, k, 128, False, seed=31)
    g_idx = torch.from_numpy(np.random.default_rng(32).permutation(k) // 128).int()
    p = L.pack_w4(q, s, z, 128, g_idx=g_idx).to(DEV)
    x = x_act(m, k, torch.bfloat16, seed=33)
    y = ops.w4a16_linear(x.to(DEV), p)
    ref = og.w4a16_gemm_ref(to_f32(x), oracle_packed(q, s, z, 128, g_idx=g_idx))
    assert_close(y.cpu(), ref, "bfloat16", what="act-order m=1024")
    with pytest.raises(ForgeError):  # the sorted weight comes with a column perm
        ops.w4a16_linear(x.to(DEV), p, config={"impl": "dequant_gemm"})


def test_graph_capture_uses_the_route_only_once_its_plan_exists():
    """A first call captured into a HIP graph takes the fused kernel (making the hipBLASLt plan inside a capture is
    not allowed); after an eager call of the same problem, a captured call takes the route.  Every replay, with eager
    work between replays, equals the eager result of the same path bit for bit."""
    m, n, k = 1024, 1536, 4096  # a problem signature no other test makes a plan for
    q, s, z = w4_parts(n, k, 128, False, seed=41)
    p = L.pack_w4(q, s, z, 128).to(DEV)
    x = x_act(m, k, torch.bfloat16, seed=42).to(DEV)
    ref = og.w4a16_gemm_ref(to_f32(x.cpu()), oracle_packed(q, s, z, 128))
    fused = ops.w4a16_linear(x, p, config={"impl": "prefill"})
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream), torch.cuda.graph(g1, stream=stream):
        y1 = ops.w4a16_linear(x, p)
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(3):
        g1.replay()
        torch.cuda.synchronize()
        assert torch.equal(y1, fused), "captured first call: not the fused kernel's bits"
        ops.w4a16_linear(x[:7], p)  # eager work between replays
    routed = ops.w4a16_linear(x, p)  # eager: makes the plan, takes the route
    assert_close(routed.cpu(), ref, "bfloat16", what="route after capture")
    assert torch.equal(routed, ops.w4a16_linear(x, p, config={"impl": "dequant_gemm"}))
    g2 = torch.cuda.CUDAGraph()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream), torch.cuda.graph(g2, stream=stream):
        y2 = ops.w4a16_linear(x, p)
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(3):
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(y2, routed), "captured call after the plan exists: not the route's bits"
        ops.w4a16_linear(x[:7], p)


def test_unaligned_x_rows_stay_off_the_route():
    """x rows K + 1 elements apart (2-byte aligned): the policy serves a 768-row call with another kernel (same bar);
    forcing the route fails instead of handing hipBLASLt rows it does not take."""
    m, n, k = 768, 512, 1024
    q, s, z = w4_parts(n, k, 128, False, seed=61)
    p = L.pack_w4(q, s, z, 128).to(DEV)
    x = x_act(m, k + 1, torch.bfloat16, seed=62).to(DEV)[:, :k]
    y = ops.w4a16_linear(x, p)
    ref = og.w4a16_gemm_ref(to_f32(x.cpu()), oracle_packed(q, s, z, 128))
    assert_close(y.cpu(), ref, "bfloat16", what="w4 unaligned x m=768")
    with pytest.raises(ForgeError):
        ops.w4a16_linear(x, p, config={"impl": "dequant_gemm"})
