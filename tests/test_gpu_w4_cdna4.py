"""GPU parity of W4A16 on the CDNA4 MFMA-fragment layout (fg_w4a16_gemm_cdna4 through w4a16_linear) against the CPU
oracle: ragged N, one / several groups, symmetric and asymmetric weights, bf16 / fp16 x, fp16 / bf16 scales, bias,
M from 1 to 64, the Llama-3-8B shapes at full size; weights repacked from portable_row at load time (a bit-exact
permutation), the packed-linear module built in that layout, and calls its kernel does not take served by the
portable copy; the LDS-ring kernel (33..64 rows, or 9..64 over K >= 8192) with and without its K-split reduce, and its
workspace check.  Bar: max|y - ref| / max|ref| <= 1e-2 plus the reference's compare() rule."""
from __future__ import annotations

import pytest
import torch

from forge_amd import _lib
from forge_amd import layouts as L
from forge_amd import ops_gemm as ops
from oracle import gemm as og
from tests._util import assert_close, gen, oracle_packed, to_f32, w4_parts, x_act

pytestmark = pytest.mark.gpu
DEV = "cuda"
ODT = {torch.bfloat16: "bfloat16", torch.float16: "float16"}


def _case(m, n, k, gs, sym, xdt, sdt=torch.float16, bias=True, seed=0):
    q, s, z = w4_parts(n, k, gs, sym, seed, sdt)
    p = ops.prepare_w4(L.pack_w4(q, s, z, gs).to(DEV), L.CDNA4_W4)
    assert p.layout.kind == L.KIND_CDNA4
    x = x_act(m, k, xdt, seed + 1)
    b = (torch.randn(n, generator=gen(seed + 2)) * 0.5).to(xdt) if bias else None
    y = ops.w4a16_linear(x.to(DEV), p, None if b is None else b.to(DEV))
    ref = og.w4a16_gemm_ref(to_f32(x), oracle_packed(q, s, z, gs), None if b is None else to_f32(b))
    return y, ref, p


@pytest.mark.parametrize("m", [1, 2, 5, 16, 17, 30, 33, 48, 64])
@pytest.mark.parametrize("n,k,gs", [(4096, 4096, 128), (1000, 2048, 256), (40, 512, -1)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_cdna4_matches_oracle(m, n, k, gs, xdt):
    sdt = torch.bfloat16 if (m + n) % 2 else torch.float16
    y, ref, _ = _case(m, n, k, gs, sym=(m % 3 == 0), xdt=xdt, sdt=sdt, seed=m + n)
    assert y.dtype == xdt and y.shape == (m, n)
    assert_close(y.cpu(), ref, ODT[xdt], what=f"cdna4 m={m} n={n} k={k} gs={gs}")


@pytest.mark.parametrize("kn", [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)])
@pytest.mark.parametrize("m", [1, 16, 64])
def test_cdna4_llama3_8b_shapes(kn, m):
    k, n = kn
    y, ref, _ = _case(m, n, k, 128, False, torch.bfloat16, bias=False, seed=k + n + m)
    assert_close(y.cpu(), ref, "bfloat16", what=f"cdna4 llama K={k} N={n} M={m}")


def test_cdna4_reproducible_and_prefill_uses_portable_copy():
    q, s, z = w4_parts(2048, 4096, 128, False, seed=5)
    p = ops.prepare_w4(L.pack_w4(q, s, z, 128).to(DEV), L.CDNA4_W4)
    x = x_act(24, 4096, seed=6).to(DEV)
    runs = [ops.w4a16_linear(x, p) for _ in range(3)]
    assert all(torch.equal(runs[0], r) for r in runs[1:])
    xb = x_act(200, 4096, seed=7)
    yb = ops.w4a16_linear(xb.to(DEV), p)  # 200 rows: the portable copy's prefill kernel
    assert_close(yb.cpu(), og.w4a16_gemm_ref(to_f32(xb), oracle_packed(q, s, z, 128)), "bfloat16", what="cdna4 M=200")


def test_cdna4_module_and_c_abi_rejections():
    n, k = 512, 1024
    q, s, z = w4_parts(n, k, 128, False, seed=8)
    mod = ops.KernelW4A16Linear.from_packed(L.pack_w4(q, s, z, 128, L.CDNA4_W4).to(DEV))
    assert mod.qweight.shape == (n // 16, 2 * k)
    x = x_act(3, k, seed=9)
    assert_close(mod(x.to(DEV)).cpu(), og.w4a16_gemm_ref(to_f32(x), oracle_packed(q, s, z, 128)), "bfloat16",
                 what="cdna4 module")
    fresh = ops.make_packed_linear("w4a16", in_features=k, out_features=n, group_size=128, sym=False,
                                   layout=L.CDNA4_W4, device=DEV)
    fresh.load_state_dict(mod.state_dict())
    assert torch.equal(fresh(x.to(DEV)), mod(x.to(DEV)))
    # fp32 scales or 65 rows are refused by the kernel's entry point
    L_ = _lib.lib()
    p = mod.packed()
    xx = x_act(65, k, seed=10).to(DEV)
    y = torch.empty(65, n, dtype=torch.bfloat16, device=DEV)
    rc = L_.fg_w4a16_gemm_cdna4(_lib.ptr(xx), k, _lib.BF16, _lib.ptr(p.qweight), p.qweight.stride(0), _lib.ptr(p.scales),
                                _lib.F16, n, _lib.ptr(p.zeros), p.zeros.stride(0), None, 0, _lib.ptr(y), n, 65, n, k, 128,
                                p.num_groups, None, 0, _lib.stream_of(xx))
    assert rc == _lib.EUNSUPPORTED and "M <= 64" in _lib.last_error()
    # the K-split plan of 64 rows over a long K needs its workspace
    assert L_.fg_w4a16_cdna4_workspace_bytes(64, n, 8192, 128) > 0
    assert L_.fg_w4a16_cdna4_workspace_bytes(16, n, 4096, 128) == 0


# The LDS-ring kernel: 33..64 rows, or 9..64 rows over K >= 8192 (N % 16 == 0); K-split plans with a reduce launch
# (small N, long K) and without (wide N), one group / several groups per step, symmetric, fp16 x, bf16 scales, bias;
# splits of 1..32 steps, so the four-wavefront loop (unrolled by its 3-stage ring) ends with 0, 1 and 2 leftover steps.
@pytest.mark.parametrize("m,n,k,gs", [(33, 2048, 4096, 128), (40, 4096, 4096, 256), (64, 1024, 2048, -1),
                                      (64, 16384, 4096, 128), (48, 512, 8192, 128), (12, 4096, 8192, 256),
                                      (16, 4096, 14336, 128), (24, 1024, 16384, -1), (64, 4096, 14336, 128),
                                      (40, 2048, 6144, 128)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_cdna4_ring_kernel(m, n, k, gs, xdt):
    sdt = torch.bfloat16 if m % 2 else torch.float16
    y, ref, _ = _case(m, n, k, gs, sym=(m % 3 == 0), xdt=xdt, sdt=sdt, bias=(m != 64), seed=m + k)
    assert_close(y.cpu(), ref, ODT[xdt], what=f"cdna4 ring m={m} n={n} k={k} gs={gs}")


def test_cdna4_ring_reproducible_and_workspace_checked():
    n, k = 4096, 14336
    q, s, z = w4_parts(n, k, 128, False, seed=11)
    p = ops.prepare_w4(L.pack_w4(q, s, z, 128).to(DEV), L.CDNA4_W4)
    x = x_act(64, k, seed=12).to(DEV)
    runs = [ops.w4a16_linear(x, p) for _ in range(3)]
    assert all(torch.equal(runs[0], r) for r in runs[1:])
    L_ = _lib.lib()
    need = L_.fg_w4a16_cdna4_workspace_bytes(64, n, k, 128)
    assert need > 0
    y = torch.empty(64, n, dtype=torch.bfloat16, device=DEV)
    args = (_lib.ptr(x), k, _lib.BF16, _lib.ptr(p.qweight), p.qweight.stride(0), _lib.ptr(p.scales), _lib.F16, n,
            _lib.ptr(p.zeros), p.zeros.stride(0), None, 0, _lib.ptr(y), n, 64, n, k, 128, p.num_groups)
    assert L_.fg_w4a16_gemm_cdna4(*args, None, 0, _lib.stream_of(x)) == _lib.EINVAL
    assert "workspace" in _lib.last_error()
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    assert L_.fg_w4a16_gemm_cdna4(*args, _lib.ptr(ws), need - 16, _lib.stream_of(x)) == _lib.EINVAL
    assert L_.fg_w4a16_gemm_cdna4(*args, _lib.ptr(ws), need, _lib.stream_of(x)) == _lib.OK
    assert torch.equal(y, runs[0])
