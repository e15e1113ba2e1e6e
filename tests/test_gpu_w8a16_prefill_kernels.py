"""GPU parity of the W8A16 prefill kernels (the reference's w8a16_linear at large M, forge/kernels/ops_gemm.py:320-346
-> gemm_wq.py:138-205 with bits=8): the ping-pong kernel's int8 form (256 x 256 tiles, fg_w4_pp.hip) and the
all-rounder's (fg_w4_big.hip).  Cases: the policy's choice from 256 rows (ping-pong once a problem has >= 160 tiles of
256 x 256; below that ping-pong with K split 2 or 4 ways when that reaches 160 tiles x splits, else the all-rounder) on
Llama-3-8B shapes; each kernel forced (tile_n = 256 / 64) on ragged shapes (one
row, M and N not multiples of the tile, bias in x's dtype / fp32 / none, per-channel and grouped fp16 / bf16 scales,
fp16 and bf16 x) and with forced K splits; "dequant_gemm" giving the same bits as "prefill"; fp32 scales and unaligned
x leaving the ping-pong kernel; graph replays; run-to-run reproducibility.

Bar: max|y - ref| / max|ref| <= 1e-2 of the fp32 oracle (forge/kernels/ref/gemm_w4a16.py:45-52 restated in
oracle/gemm.py) plus the reference's compare() rule.
"""
from __future__ import annotations

import pytest
import torch

from forge_amd import layouts as L
from forge_amd import ops_gemm as ops
from oracle import gemm as og
from tests._util import assert_close, gen, to_f32, x_act

pytestmark = pytest.mark.gpu
DEV = "cuda"
ODT = {torch.bfloat16: "bfloat16", torch.float16: "float16"}
KERNEL = {256: "w4_pp_kernel", 64: "w4_big_kernel"}


def _run(m, n, k, gs, xdt, bdt, *, seed, sdt=torch.float16, config=None):
    g = gen(seed)
    q = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand(n, L.num_groups(k, gs), generator=g) * 0.018 + 0.002).to(sdt)
    p = L.pack_w8(q, s, gs).to(DEV)
    x = x_act(m, k, xdt, seed + 1)
    b = None if bdt is None else (torch.randn(n, generator=gen(seed + 2)) * 0.5).to(bdt)
    bd = None if b is None else b.to(DEV)
    y = ops.w8a16_linear(x.to(DEV), p, bd, config=config)
    kern = ops.last_kernel()
    assert ops.last_path("w8a16_linear") == "hip" and y.dtype == xdt and y.shape == (m, n)
    ref = og.w8a16_gemm_ref(to_f32(x), og.pack_w8(q.numpy(), s.float().numpy(), gs), None if b is None else to_f32(b))
    return y, ref, kern, (x.to(DEV), p, bd)


@pytest.mark.parametrize("m,k,n,gs,xdt,bdt,expect", [
    (768, 4096, 28672, -1, torch.bfloat16, torch.bfloat16, "w4_pp_kernel<bf16,w8> 256x256 splits=1"),  # 336 tiles
    (4096, 4096, 4096, 128, torch.float16, torch.float32, "w4_pp_kernel<f16,w8> 256x256 splits=1"),    # 256 tiles
    (1024, 4096, 6144, -1, torch.bfloat16, torch.bfloat16, "w4_pp_kernel<bf16,w8> 256x256 splits=2"),  # 96 tiles
    (1024, 14336, 4096, -1, torch.bfloat16, None, "w4_pp_kernel<bf16,w8> 256x256 splits=4"),           # 64 tiles
    (2048, 4096, 2048, 64, torch.float16, torch.float16, "w4_pp_kernel<f16,w8> 256x256 splits=4"),     # 64 tiles
    (512, 4096, 4096, -1, torch.bfloat16, torch.bfloat16, "w4_big_kernel"),                            # 32 tiles
    (300, 14336, 4096, 128, torch.float16, None, "w4_big_kernel"),                                     # 32 tiles
])
def test_policy_choice_from_256_rows(m, k, n, gs, xdt, bdt, expect):
    y, ref, kern, (x, p, bd) = _run(m, n, k, gs, xdt, bdt, seed=m + n)
    assert kern.startswith(expect) and "w8" in kern, kern
    assert_close(y.cpu(), ref, ODT[xdt], what=f"w8a16 prefill m={m} k={k} n={n} gs={gs}")
    assert torch.equal(y, ops.w8a16_linear(x, p, bd)), "not reproducible run to run"
    assert torch.equal(y, ops.w8a16_linear(x, p, bd, config={"impl": "dequant_gemm"}))


RAGGED = [  # m, k, n, gs, xdt, bdt, sdt
    (300, 1024, 520, 128, torch.bfloat16, torch.bfloat16, torch.float16),
    (1, 512, 128, -1, torch.float16, None, torch.float16),
    (257, 4096, 4104, -1, torch.bfloat16, torch.float32, torch.bfloat16),
    (700, 2048, 1032, 64, torch.float16, torch.float16, torch.float16),
    (513, 1536, 776, 192, torch.bfloat16, None, torch.bfloat16),
]


@pytest.mark.parametrize("tile_n", [256, 64])
@pytest.mark.parametrize("m,k,n,gs,xdt,bdt,sdt", RAGGED)
def test_forced_kernel_ragged(tile_n, m, k, n, gs, xdt, bdt, sdt):
    y, ref, kern, _ = _run(m, n, k, gs, xdt, bdt, seed=m + k + tile_n, sdt=sdt,
                           config={"impl": "prefill", "tile_n": tile_n})
    assert kern.startswith(KERNEL[tile_n]), kern
    assert_close(y.cpu(), ref, ODT[xdt], what=f"w8 {KERNEL[tile_n]} m={m} k={k} n={n} gs={gs}")


@pytest.mark.parametrize("tile_n,split", [(256, 3), (256, 8), (64, 2)])
def test_forced_k_splits(tile_n, split):
    y, ref, kern, (x, p, bd) = _run(320, 1032, 4096, 128, torch.bfloat16, torch.bfloat16, seed=80 + split,
                                    config={"impl": "prefill", "tile_n": tile_n, "split_k": split})
    assert kern.startswith(KERNEL[tile_n]) and f"splits={split}" in kern, kern
    assert_close(y.cpu(), ref, "bfloat16", what=kern)


@pytest.mark.parametrize("m,gs,xdt,bdt,sdt", [(64, -1, torch.bfloat16, torch.float32, torch.float16),
                                              (5, 96, torch.float16, None, torch.bfloat16),
                                              (300, 128, torch.bfloat16, torch.bfloat16, torch.float32)])
def test_dequant_gemm_names_the_prefill_kernels(m, gs, xdt, bdt, sdt):
    """The reference's dequant_matmul at any M: the prefill kernels (fp32 scales and groups of 96 take the
    all-rounder)."""
    y, ref, kern, (x, p, bd) = _run(m, 2048, 1536, gs, xdt, bdt, seed=m, sdt=sdt, config={"impl": "dequant_gemm"})
    assert kern.startswith(("w4_pp_kernel", "w4_big_kernel")), kern
    assert_close(y.cpu(), ref, ODT[xdt], what=f"w8a16 dequant_gemm m={m} gs={gs}")
    assert torch.equal(y, ops.w8a16_linear(x, p, bd, config={"impl": "prefill"}))


def test_graph_replays():
    """A captured ping-pong call replayed three times, with eager work between replays, equals the eager result."""
    m, n, k = 1024, 1792, 4096
    _, _, _, (_, p, _) = _run(8, n, k, 128, torch.bfloat16, None, seed=41)
    x = x_act(m, k, torch.bfloat16, 42).to(DEV)
    cfg = {"impl": "prefill", "tile_n": 256}
    eager = ops.w8a16_linear(x, p, config=cfg)
    assert ops.last_kernel().startswith("w4_pp_kernel")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream), torch.cuda.graph(g, stream=stream):
        yg = ops.w8a16_linear(x, p, config=cfg)
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, eager), "replay differs from the eager call"
        ops.w8a16_linear(x[:7], p)


def test_unaligned_x_rows():
    """x rows K + 1 elements apart (2-byte aligned): a kernel that takes them serves the 768-row call."""
    m, n, k = 768, 512, 1024
    g = gen(51)
    q = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand(n, 1, generator=g) * 0.018 + 0.002).half()
    p = L.pack_w8(q, s, -1).to(DEV)
    x = x_act(m, k + 1, torch.bfloat16, 52).to(DEV)[:, :k]
    y = ops.w8a16_linear(x, p)
    assert not ops.last_kernel().startswith("w4_pp_kernel")
    ref = og.w8a16_gemm_ref(to_f32(x.cpu()), og.pack_w8(q.numpy(), s.float().numpy(), -1), None)
    assert_close(y.cpu(), ref, "bfloat16", what="w8a16 unaligned x m=768")
