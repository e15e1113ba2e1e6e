"""GPU parity of W8A16's dequantise + library GEMM route: the int8 weights dequantised once into the workspace by the
dense W8 dequantisation kernel (q * s in fp32 rounded once to x's dtype, the value the fused prefill kernel stores
into LDS), then hipBLASLt's bf16 / fp16 GEMM with the bias in its epilogue.  The policy takes it from 768 rows;
forced through config={"impl": "dequant_gemm"} at any M.  Cases: bf16 / fp16 x, per-channel and grouped 16-bit / fp32
scales, bias in x's dtype / fp32 / none, a bias type the route does not take (the fused kernel serves the call),
weights large enough to go through in two channel chunks, graph capture before and after the plan exists, run-to-run
reproducibility.

Bar: max|y - ref| / max|ref| <= 1e-2 of the fp32 oracle (forge/kernels/ref/gemm_w4a16.py:45-52 restated in
oracle/gemm.py) plus the reference's compare() rule.
"""
from __future__ import annotations

import pytest
import torch

from forge_amd import layouts as L
from forge_amd import ops_gemm as ops
from forge_amd.errors import ForgeError
from oracle import gemm as og
from tests._util import assert_close, gen, to_f32, x_act

pytestmark = pytest.mark.gpu
DEV = "cuda"
ODT = {torch.bfloat16: "bfloat16", torch.float16: "float16"}


def _run(m, n, k, gs, xdt, bdt, *, seed, sdt=torch.float16, config=None):
    g = gen(seed)
    q = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand(n, L.num_groups(k, gs), generator=g) * 0.018 + 0.002).to(sdt)
    p = L.pack_w8(q, s, gs).to(DEV)
    x = x_act(m, k, xdt, seed + 1)
    b = None if bdt is None else (torch.randn(n, generator=gen(seed + 2)) * 0.5).to(bdt)
    bd = None if b is None else b.to(DEV)
    y = ops.w8a16_linear(x.to(DEV), p, bd, config=config)
    assert ops.last_path("w8a16_linear") == "hip" and y.dtype == xdt and y.shape == (m, n)
    ref = og.w8a16_gemm_ref(to_f32(x), og.pack_w8(q.numpy(), s.float().numpy(), gs), None if b is None else to_f32(b))
    return y, ref, (x.to(DEV), p, bd)


@pytest.mark.parametrize("m,k,n,gs,xdt,bdt", [
    (768, 4096, 28672, -1, torch.bfloat16, torch.bfloat16),
    (1024, 4096, 6144, -1, torch.bfloat16, torch.bfloat16),
    (1500, 4096, 4096, 128, torch.float16, torch.float32),
    (1024, 14336, 4096, -1, torch.bfloat16, None),
    (2048, 4096, 2048, 64, torch.float16, torch.float16),
])
def test_policy_takes_the_route_from_768_rows(m, k, n, gs, xdt, bdt):
    y, ref, (x, p, bd) = _run(m, n, k, gs, xdt, bdt, seed=m + n)
    assert_close(y.cpu(), ref, ODT[xdt], what=f"w8a16 dequant+gemm m={m} k={k} n={n} gs={gs}")
    assert torch.equal(y, ops.w8a16_linear(x, p, bd)), "not reproducible run to run"
    assert torch.equal(y, ops.w8a16_linear(x, p, bd, config={"impl": "dequant_gemm"}))


@pytest.mark.parametrize("m,gs,xdt,bdt,sdt", [(64, -1, torch.bfloat16, torch.float32, torch.float16),
                                              (5, 96, torch.float16, None, torch.bfloat16),
                                              (300, 128, torch.bfloat16, torch.bfloat16, torch.float32)])
def test_forced_route_at_few_rows(m, gs, xdt, bdt, sdt):
    y, ref, _ = _run(m, 2048, 1536, gs, xdt, bdt, seed=m, sdt=sdt, config={"impl": "dequant_gemm"})
    assert_close(y.cpu(), ref, ODT[xdt], what=f"forced w8a16 dequant+gemm m={m} gs={gs}")


def test_route_level_with_the_fused_prefill_kernel():
    """Both paths multiply the same rounded weights; only the fp32 summation order differs."""
    y, ref, (x, p, bd) = _run(1024, 4096, 4096, 128, torch.bfloat16, torch.bfloat16, seed=7)
    fused = ops.w8a16_linear(x, p, bd, config={"impl": "prefill"})
    assert_close(fused.cpu(), ref, "bfloat16", what="fused prefill m=1024")
    err = (y.float() - fused.float()).abs().max().item() / fused.float().abs().max().item()
    assert err < 1e-2, err


def test_bias_type_the_route_does_not_take_falls_back():
    """bf16 x with an fp16 bias: the fused prefill kernel serves the call (same bar); forcing the route fails."""
    y, ref, _ = _run(1024, 4096, 4096, -1, torch.bfloat16, torch.float16, seed=11)
    assert_close(y.cpu(), ref, "bfloat16", what="fp16 bias fallback")
    with pytest.raises(ForgeError):
        _run(64, 256, 512, -1, torch.bfloat16, torch.float16, seed=12, config={"impl": "dequant_gemm"})


def test_two_channel_chunks():
    """33024 x 8192 weights dequantise to 541 MB, over the 512 MB chunk: two dequantise + GEMM passes."""
    y, ref, _ = _run(64, 33024, 8192, -1, torch.bfloat16, torch.bfloat16, seed=21, config={"impl": "dequant_gemm"})
    assert_close(y.cpu(), ref, "bfloat16", what="two chunks")


def test_graph_capture_uses_the_route_only_once_its_plan_exists():
    """A first call captured into a HIP graph takes the fused kernel (making the hipBLASLt plan inside a capture is
    not allowed); after an eager call of the same problem, a captured call takes the route.  Every replay, with eager
    work between replays, equals the eager result of the same path bit for bit."""
    m, n, k = 1024, 1792, 4096  # a problem signature no other test makes a plan for
    _, ref, (x, p, _) = _run(8, n, k, 128, torch.bfloat16, None, seed=41)
    x = x_act(m, k, torch.bfloat16, 42).to(DEV)
    fused = ops.w8a16_linear(x, p, config={"impl": "prefill"})
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream), torch.cuda.graph(g1, stream=stream):
        y1 = ops.w8a16_linear(x, p)
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(3):
        g1.replay()
        torch.cuda.synchronize()
        assert torch.equal(y1, fused), "captured first call: not the fused kernel's bits"
        ops.w8a16_linear(x[:7], p)  # eager work between replays
    routed = ops.w8a16_linear(x, p)  # eager: makes the plan, takes the route
    err = (routed.float() - fused.float()).abs().max().item() / fused.float().abs().max().item()
    assert err < 1e-2, err
    assert torch.equal(routed, ops.w8a16_linear(x, p, config={"impl": "dequant_gemm"}))
    g2 = torch.cuda.CUDAGraph()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream), torch.cuda.graph(g2, stream=stream):
        y2 = ops.w8a16_linear(x, p)
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(3):
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(y2, routed), "captured call after the plan exists: not the route's bits"
        ops.w8a16_linear(x[:7], p)


def test_unaligned_x_rows_stay_off_the_route():
    """x rows K + 1 elements apart (2-byte aligned): the policy serves a 768-row call with another kernel (same bar);
    forcing the route fails instead of handing hipBLASLt rows it does not take."""
    m, n, k = 768, 512, 1024
    g = gen(51)
    q = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand(n, 1, generator=g) * 0.018 + 0.002).half()
    p = L.pack_w8(q, s, -1).to(DEV)
    x = x_act(m, k + 1, torch.bfloat16, 52).to(DEV)[:, :k]
    y = ops.w8a16_linear(x, p)
    ref = og.w8a16_gemm_ref(to_f32(x.cpu()), og.pack_w8(q.numpy(), s.float().numpy(), -1), None)
    assert_close(y.cpu(), ref, "bfloat16", what="w8a16 unaligned x m=768")
    with pytest.raises(ForgeError):
        ops.w8a16_linear(x, p, config={"impl": "dequant_gemm"})
