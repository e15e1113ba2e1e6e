"""GPU parity of the W4A16 prefill kernels, the hand-written side of the reference's large-M paths
(forge/kernels/triton/gemm_w4_dequant.py:194-256 w4_dequant_matmul, gemm_w4a16.py:69-153): the ping-pong kernel
(256 x 256 tiles, fg_w4_pp.hip), the producer / consumer kernel (256 x 128, fg_w4_pc.hip) and the all-rounder
(fg_w4_big.hip).  Cases: the policy's choice from 256 rows (ping-pong once a problem has >= 160 tiles of 256 x 256,
else producer / consumer) on Llama-3-8B shapes; each kernel forced (tile_n = 256 / 128 / 64) on ragged shapes (M and N
not multiples of the tile, one row, bias in x's dtype / fp32 / none, symmetric and asymmetric weights, one group and
groups of 64 / 128, fp16 and bf16 x and scales) and with forced K splits; "dequant_gemm" (the reference's
dequant_matmul) giving the same bits as "prefill"; act-order weights, fp32 scales and unaligned x leaving the fast
kernels; graph replays; run-to-run reproducibility.

Bar: max|y - ref| / max|ref| <= 1e-2 of the fp32 oracle (oracle/gemm.py) plus the reference's compare() rule.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from forge_amd import layouts as L
from forge_amd import ops_gemm as ops
from oracle import gemm as og
from tests._util import assert_close, gen, oracle_packed, to_f32, w4_parts, x_act

pytestmark = pytest.mark.gpu
DEV = "cuda"
ODT = {torch.bfloat16: "bfloat16", torch.float16: "float16"}
KERNEL = {256: "w4_pp_kernel", 128: "w4_pc_kernel", 64: "w4_big_kernel"}


def _run(m, n, k, xdt, bdt, *, seed, gs=128, config=None, sym=False, sdt=torch.float16):
    q, s, z = w4_parts(n, k, gs, sym, seed=seed, scale_dtype=sdt)
    p = L.pack_w4(q, s, z, gs).to(DEV)
    x = x_act(m, k, xdt, seed=seed + 1)
    b = None if bdt is None else (torch.randn(n, generator=gen(seed + 2)) * 0.5).to(bdt)
    bd = None if b is None else b.to(DEV)
    y = ops.w4a16_linear(x.to(DEV), p, bd, config=config)
    kern = ops.last_kernel()
    assert ops.last_path("w4a16_linear") == "hip" and y.dtype == xdt and y.shape == (m, n)
    ref = og.w4a16_gemm_ref(to_f32(x), oracle_packed(q, s, z, gs), None if b is None else to_f32(b))
    return y, ref, kern, (x.to(DEV), p, bd)


@pytest.mark.parametrize("m,k,n,xdt,bdt,expect", [
    (768, 4096, 28672, torch.bfloat16, torch.bfloat16, "w4_pp_kernel"),   # 336 tiles
    (4096, 4096, 4096, torch.float16, torch.float16, "w4_pp_kernel"),     # 256 tiles
    (1024, 4096, 6144, torch.bfloat16, torch.bfloat16, "w4_pc_kernel"),   # 96 tiles
    (1500, 4096, 6144, torch.float16, torch.float32, "w4_pc_kernel"),
    (1024, 14336, 4096, torch.bfloat16, None, "w4_pc_kernel"),
    (256, 4096, 28672, torch.bfloat16, None, "w4_pc_kernel"),             # 112 tiles
])
def test_policy_choice_from_256_rows(m, k, n, xdt, bdt, expect):
    y, ref, kern, (x, p, bd) = _run(m, n, k, xdt, bdt, seed=m + n)
    assert kern.startswith(expect), kern
    assert_close(y.cpu(), ref, ODT[xdt], what=f"prefill m={m} k={k} n={n}")
    assert torch.equal(y, ops.w4a16_linear(x, p, bd)), "not reproducible run to run"
    # the reference's dequant_matmul names the same kernels
    assert torch.equal(y, ops.w4a16_linear(x, p, bd, config={"impl": "dequant_gemm"}))
    assert torch.equal(y, ops.w4a16_linear(x, p, bd, config={"impl": "dequant_matmul"}))


RAGGED = [  # m, k, n, gs, xdt, bdt, sym, sdt
    (300, 1024, 520, 128, torch.bfloat16, torch.bfloat16, False, torch.float16),
    (1, 512, 128, 128, torch.float16, None, True, torch.float16),
    (257, 4096, 4104, -1, torch.bfloat16, torch.float32, False, torch.bfloat16),
    (700, 2048, 1032, 64, torch.float16, torch.float16, False, torch.float16),
    (513, 1536, 776, 64, torch.bfloat16, None, True, torch.bfloat16),
]


@pytest.mark.parametrize("tile_n", [256, 128, 64])
@pytest.mark.parametrize("m,k,n,gs,xdt,bdt,sym,sdt", RAGGED)
def test_forced_kernel_ragged(tile_n, m, k, n, gs, xdt, bdt, sym, sdt):
    y, ref, kern, _ = _run(m, n, k, xdt, bdt, seed=m + k + tile_n, gs=gs, sym=sym, sdt=sdt,
                           config={"impl": "prefill", "tile_n": tile_n})
    assert kern.startswith(KERNEL[tile_n]), kern
    assert_close(y.cpu(), ref, ODT[xdt], what=f"{KERNEL[tile_n]} m={m} k={k} n={n} gs={gs}")


@pytest.mark.parametrize("tile_n,split", [(256, 3), (256, 8), (128, 5), (64, 2)])
def test_forced_k_splits(tile_n, split):
    """Fixed-order split-K partials in the caller's workspace, reduced with the bias."""
    y, ref, kern, (x, p, bd) = _run(320, 1032, 4096, torch.bfloat16, torch.bfloat16, seed=70 + split,
                                    config={"impl": "prefill", "tile_n": tile_n, "split_k": split})
    assert kern.startswith(KERNEL[tile_n]) and f"splits={split}" in kern, kern
    assert_close(y.cpu(), ref, "bfloat16", what=f"{kern}")
    assert torch.equal(y, ops.w4a16_linear(x, p, bd, config={"impl": "prefill", "tile_n": tile_n, "split_k": split}))


def test_act_order_and_fp32_scales_leave_the_fast_kernels():
    n, k, m = 1024, 2048, 1024
    q, s, z = w4_parts(n, k, 128, False, seed=31)
    g_idx = torch.from_numpy(np.random.default_rng(32).permutation(k) // 128).int()
    p = L.pack_w4(q, s, z, 128, g_idx=g_idx).to(DEV)
    x = x_act(m, k, torch.bfloat16, seed=33)
    y = ops.w4a16_linear(x.to(DEV), p)
    kern = ops.last_kernel()
    assert not kern.startswith(("w4_pp_kernel", "w4_pc_kernel")), kern  # the sorted weight comes with a column perm
    ref = og.w4a16_gemm_ref(to_f32(x), oracle_packed(q, s, z, 128, g_idx=g_idx))
    assert_close(y.cpu(), ref, "bfloat16", what="act-order m=1024")
    y, ref, kern, _ = _run(1024, 4096, 4096, torch.bfloat16, None, seed=34, sdt=torch.float32)
    assert not kern.startswith(("w4_pp_kernel", "w4_pc_kernel")), kern
    assert_close(y.cpu(), ref, "bfloat16", what="fp32 scales m=1024")


def test_unaligned_x_rows():
    """x rows K + 1 elements apart (2-byte aligned): the policy serves a 768-row call with a kernel that takes them."""
    m, n, k = 768, 512, 1024
    q, s, z = w4_parts(n, k, 128, False, seed=61)
    p = L.pack_w4(q, s, z, 128).to(DEV)
    x = x_act(m, k + 1, torch.bfloat16, seed=62).to(DEV)[:, :k]
    y = ops.w4a16_linear(x, p)
    ref = og.w4a16_gemm_ref(to_f32(x.cpu()), oracle_packed(q, s, z, 128))
    assert_close(y.cpu(), ref, "bfloat16", what="w4 unaligned x m=768")


@pytest.mark.parametrize("tile_n", [256, 128])
def test_graph_replays(tile_n):
    """A captured call replayed three times, with eager work between replays, equals the eager result bit for bit."""
    m, n, k = 1024, 2048, 4096
    q, s, z = w4_parts(n, k, 128, False, seed=41)
    p = L.pack_w4(q, s, z, 128).to(DEV)
    x = x_act(m, k, torch.bfloat16, seed=42).to(DEV)
    cfg = {"impl": "prefill", "tile_n": tile_n}
    eager = ops.w4a16_linear(x, p, config=cfg)
    assert ops.last_kernel().startswith(KERNEL[tile_n])
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream), torch.cuda.graph(g, stream=stream):
        yg = ops.w4a16_linear(x, p, config=cfg)
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, eager), "replay differs from the eager call"
        ops.w4a16_linear(x[:7], p)  # eager work between replays
    ref = og.w4a16_gemm_ref(to_f32(x.cpu()), oracle_packed(q, s, z, 128))
    assert_close(eager.cpu(), ref, "bfloat16", what=f"graph {KERNEL[tile_n]}")
