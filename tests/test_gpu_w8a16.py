"""GPU parity of W8A16 (fg_w8a16_gemm through the C ABI: decode GEMV, LDS-ring and skinny MFMA, dequantise-to-LDS
prefill and generic kernels)
against the CPU oracle (forge/kernels/ref/gemm_w4a16.py:45-52 restated in oracle/gemm.py).  Bar: max|y - ref| /
max|ref| <= 1e-2 of the fp32 oracle and the reference's compare() rule for bf16 / fp16 outputs."""
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


def _w8(n, k, gs, seed, sdt=torch.float16):
    g = gen(seed)
    q = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    ng = L.num_groups(k, gs)
    s = (torch.rand(n, ng, generator=g) * 0.018 + 0.002).to(sdt)
    return q, s


def _case(m, n, k, gs, xdt, *, sdt=torch.float16, bias=True, seed=0, config=None):
    q, s = _w8(n, k, gs, seed, sdt)
    p = L.pack_w8(q, s, gs).to(DEV)
    x = x_act(m, k, xdt, seed + 1)
    b = (torch.randn(n, generator=gen(seed + 2)) * 0.5).to(xdt) if bias else None
    y = ops.w8a16_linear(x.to(DEV), p, None if b is None else b.to(DEV), config=config)
    assert ops.last_path("w8a16_linear") == "hip" and y.dtype == xdt and y.shape == (m, n)
    ref = og.w8a16_gemm_ref(to_f32(x), og.pack_w8(q.numpy(), s.float().numpy(), gs),
                            None if b is None else to_f32(b))
    return y, ref


@pytest.mark.parametrize("m", [1, 4, 16, 33, 64])
@pytest.mark.parametrize("n,k,gs", [(4096, 4096, -1), (777, 2048, 128), (1030, 1024, 256)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_skinny_matches_oracle(m, n, k, gs, xdt):
    sdt = torch.bfloat16 if m % 2 else torch.float16
    y, ref = _case(m, n, k, gs, xdt, sdt=sdt, seed=m + n, config={"impl": "mfma"})
    assert_close(y.cpu(), ref, ODT[xdt], what=f"w8a16 skinny m={m} n={n} k={k} gs={gs}")


# The LDS-ring kernel through the automatic policy (17..64 rows, and 3..16 over N >= 16384 or K >= 8192), one case per
# launch shape: one row block (K split 16 ways + reduce / whole K), two, four on four wavefronts, two and four on eight
# wavefronts (row sums shared through LDS; wide N / long K), one group per row, bias or not.
@pytest.mark.parametrize("m,n,k,gs", [(5, 16384, 1024, 128), (12, 1024, 8192, 256), (17, 2048, 2048, -1),
                                      (40, 4096, 4096, 128), (64, 16384, 1024, 128), (33, 6144, 2048, 128),
                                      (64, 1024, 8192, 128), (24, 6144, 1024, 128)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_ring_matches_oracle(m, n, k, gs, xdt):
    sdt = torch.bfloat16 if m % 2 else torch.float16
    y, ref = _case(m, n, k, gs, xdt, sdt=sdt, bias=(m % 3 != 0), seed=m + n + k)
    assert_close(y.cpu(), ref, ODT[xdt], what=f"w8a16 ring m={m} n={n} k={k} gs={gs}")


def test_ring_reproducible_and_level_with_skinny():
    q, s = _w8(6144, 2048, 128, seed=81)
    p = L.pack_w8(q, s, 128).to(DEV)
    x = x_act(48, 2048, seed=82).to(DEV)
    runs = [ops.w8a16_linear(x, p) for _ in range(3)]
    assert all(torch.equal(runs[0], r) for r in runs[1:])
    ref = og.w8a16_gemm_ref(to_f32(x.cpu()), og.pack_w8(q.numpy(), s.float().numpy(), 128))
    assert_close(runs[0].cpu(), ref, "bfloat16", what="w8a16 ring m=48")
    assert_close(ops.w8a16_linear(x, p, config={"impl": "mfma"}).cpu(), ref, "bfloat16", what="w8a16 skinny m=48")


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k,gs", [(4096, 4096, -1), (776, 2048, 128), (1032, 1024, 256), (512, 960, 48),
                                    (264, 20480, 128), (8, 16, 16), (1024, 8192, 128), (520, 14336, -1)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_gemv_matches_oracle(m, n, k, gs, xdt):
    """The split-K decode GEMV forced (one, two and four chunks per lane, group sizes that are not powers of two, a K
    of one chunk), against the oracle; for one or two rows the policy takes it too and gives the same bits."""
    sdt = torch.bfloat16 if (m + n) % 2 else torch.float16
    if m > 2 and k > 16384:  # four rows of x: at most 8 slices of 1024 columns; the policy takes the skinny kernel
        with pytest.raises(ForgeError):
            _case(m, n, k, gs, xdt, sdt=sdt, seed=m + n + k, config={"impl": "gemv"})
        y2, ref = _case(m, n, k, gs, xdt, sdt=sdt, seed=m + n + k)
        assert_close(y2.cpu(), ref, ODT[xdt], what=f"w8a16 policy m={m} n={n} k={k} gs={gs}")
        return
    y, ref = _case(m, n, k, gs, xdt, sdt=sdt, seed=m + n + k, config={"impl": "gemv"})
    assert_close(y.cpu(), ref, ODT[xdt], what=f"w8a16 gemv m={m} n={n} k={k} gs={gs}")
    y2, _ = _case(m, n, k, gs, xdt, sdt=sdt, seed=m + n + k)
    if m <= 2:  # the policy's own choice for one or two rows
        assert torch.equal(y, y2), f"gemv m={m} n={n}: policy differs from the forced GEMV"
    else:
        assert_close(y2.cpu(), ref, ODT[xdt], what=f"w8a16 policy m={m} n={n} k={k} gs={gs}")


def test_gemv_extremes_and_rejects():
    """Weights at -128 and 127 with large x (exact products, fp32 sums), NaN / inf in x propagate, run-to-run bits;
    the forced GEMV rejects 5 rows and channel counts that its wavefronts do not divide."""
    n, k = 1024, 4096
    q = torch.full((n, k), 127, dtype=torch.int8)
    q[::2] = -128
    s = torch.full((n, 1), 0.5, dtype=torch.float16)
    p = L.pack_w8(q, s, -1).to(DEV)
    x = (torch.randn(2, k, generator=gen(81)) * 100).bfloat16()
    x[1, 7] = float("nan")
    y = ops.w8a16_linear(x.to(DEV), p, config={"impl": "gemv"})
    ref = og.w8a16_gemm_ref(to_f32(x[:1]), og.pack_w8(q.numpy(), s.float().numpy(), -1))
    assert_close(y[:1].cpu(), ref, "bfloat16", what="gemv extremes")
    assert torch.isnan(y[1].float()).all()
    assert all(torch.equal(y[:1], ops.w8a16_linear(x.to(DEV), p, config={"impl": "gemv"})[:1]) for _ in range(3))
    with pytest.raises(ForgeError):
        ops.w8a16_linear(x_act(5, k, seed=82).to(DEV), p, config={"impl": "gemv"})
    q2, s2 = _w8(100, 256, -1, seed=83)
    with pytest.raises(ForgeError):
        ops.w8a16_linear(x_act(1, 256, seed=84).to(DEV), L.pack_w8(q2, s2, -1).to(DEV), config={"impl": "gemv"})


# (200, 1024, 8192) and (390, 4096, 14336): 8-bit weights over K >= 8192 from 129 rows, where the plan takes 256-row
# tiles (ragged last row tile, K split 16 / 5 ways)
@pytest.mark.parametrize("m,n,k,gs", [(65, 256, 512, 32), (128, 777, 1024, -1), (300, 2048, 2048, 128),
                                      (200, 1024, 8192, 128), (390, 4096, 14336, -1)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_prefill_matches_oracle(m, n, k, gs, xdt):
    y, ref = _case(m, n, k, gs, xdt, seed=m + k, config={"impl": "prefill"})
    assert_close(y.cpu(), ref, ODT[xdt], what=f"w8a16 prefill m={m} n={n} k={k}")
    y2, _ = _case(m, n, k, gs, xdt, seed=m + k)  # policy
    assert_close(y2.cpu(), ref, ODT[xdt], what=f"w8a16 policy m={m} n={n} k={k}")


@pytest.mark.parametrize("m,n,k,gs,sdt", [(3, 333, 100, 8, torch.float16), (70, 129, 1000, 40, torch.float32),
                                          (1, 64, 4096, 128, torch.float32)])
def test_generic_and_odd_shapes(m, n, k, gs, sdt):
    y, ref = _case(m, n, k, gs, torch.bfloat16, sdt=sdt, seed=k, config={"impl": "generic"})
    assert_close(y.cpu(), ref, "bfloat16", what=f"w8a16 generic m={m} n={n} k={k}")
    y2, _ = _case(m, n, k, gs, torch.bfloat16, sdt=sdt, seed=k)  # the policy falls back where it must
    assert_close(y2.cpu(), ref, "bfloat16", what=f"w8a16 policy odd m={m} n={n} k={k}")


def test_split_k_reproducible_rejects_and_modules():
    q, s = _w8(1024, 2048, 128, seed=71)
    p = L.pack_w8(q, s, 128).to(DEV)
    x = x_act(200, 2048, seed=72).to(DEV)
    runs = [ops.w8a16_linear(x, p, config={"impl": "prefill", "split_k": 3}) for _ in range(3)]
    assert all(torch.equal(runs[0], r) for r in runs[1:])
    ref = og.w8a16_gemm_ref(to_f32(x.cpu()), og.pack_w8(q.numpy(), s.float().numpy(), 128))
    assert_close(runs[0].cpu(), ref, "bfloat16", what="w8a16 split-K")
    x16 = x_act(16, 2048, seed=73).to(DEV)
    r16 = [ops.w8a16_linear(x16, p) for _ in range(3)]
    assert all(torch.equal(r16[0], r) for r in r16[1:])
    with pytest.raises(ForgeError):  # skinny kernel forced on K % 128 != 0
        q2, s2 = _w8(64, 1000, -1, seed=74)
        ops.w8a16_linear(x_act(4, 1000, seed=75).to(DEV), L.pack_w8(q2, s2, -1).to(DEV), config={"impl": "mfma"})
    lin = torch.nn.Linear(256, 96).to(DEV)
    m = ops.make_packed_linear("w8a16", lin, group_size=128)
    xi = x_act(5, 256, seed=76).to(DEV)
    assert_close(m(xi).float().cpu(), (xi.float() @ m.dequantize().t() + lin.bias.float()).detach().cpu().numpy(),
                 "bfloat16", what="module")


@pytest.mark.parametrize("kn", [(4096, 6144), (4096, 28672), (14336, 4096)])
@pytest.mark.parametrize("m", [1, 16, 64])
def test_llama3_8b_shapes(kn, m):
    k, n = kn
    y, ref = _case(m, n, k, -1, torch.bfloat16, bias=False, seed=k + n)
    assert_close(y.cpu(), ref, "bfloat16", what=f"w8a16 llama K={k} N={n} M={m}")
