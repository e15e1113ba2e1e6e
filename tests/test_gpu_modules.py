"""GPU forward of the packed-linear modules the model loader swaps in (KernelW4A16Linear, KernelFp8Linear,
KernelInt8Linear and make_packed_linear; reference forge/kernels/ops_gemm.py:769-961,1025-1068): built from packed
data, from a dense nn.Linear, and from a state dict loaded into a module made by shape (act-order included), each
against the CPU oracle on the same inputs.

Bars: W4A16 / FP8 within max|y - ref| / max|ref| <= 1e-2 plus compare(); INT8 weight codes, scales and the bf16
output bit-exact; FP8 weight codes and scales bit-exact; a module rebuilt from a state dict equals the original bit for
bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from forge_amd import layouts as L
from forge_amd import ops_gemm as ops
from oracle import gemm as og
from tests._util import assert_close, fp8_codes, gen, oracle_packed, to_f32, w4_parts, x_act

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("m", [1, 16, 200])
@pytest.mark.parametrize("act_order", [False, True])
def test_w4a16_module_from_packed_and_state_dict(m, act_order):
    n, k, gs = 1536, 2048, 128
    q, s, z = w4_parts(n, k, gs, False, seed=m + 5)
    g_idx = (torch.arange(k) // gs)[torch.randperm(k, generator=gen(m))].to(torch.int32) if act_order else None
    b = (torch.randn(n, generator=gen(m + 1)) * 0.5).half()
    a = ops.KernelW4A16Linear.from_packed(L.pack_w4(q, s, z, gs, g_idx=g_idx).to(DEV), b.to(DEV))
    x = x_act(m, k, torch.bfloat16, seed=m + 2)
    y = a(x.to(DEV))
    assert ops.last_path("w4a16_linear") == "hip" and y.dtype == torch.bfloat16
    ref = og.w4a16_gemm_ref(to_f32(x), oracle_packed(q, s, z, gs, g_idx), to_f32(b.bfloat16()))
    assert_close(y.cpu(), ref, "bfloat16", what=f"KernelW4A16Linear m={m} act_order={act_order}")
    # a module made by shape, then loaded from the state dict (the loader's route), gives the same bits
    fresh = ops.make_packed_linear("w4a16", in_features=k, out_features=n, bias=torch.zeros(n), group_size=gs,
                                   sym=False, has_g_idx=act_order, dtype=torch.float16, device=DEV)
    fresh.load_state_dict(a.state_dict())
    assert torch.equal(fresh(x.to(DEV)), y)


def test_w4a16_module_from_dense_matches_its_own_dequantisation():
    lin = torch.nn.Linear(1024, 384).to(DEV)
    mod = ops.make_packed_linear("w4a16", lin, group_size=128, sym=False)
    x = x_act(8, 1024, torch.float16, seed=3).to(DEV)
    y = mod(x)
    # the module's packed weight, dequantised by the oracle from its unpacked parts
    q, s, z = L.unpack_w4(mod.packed())
    ref = og.w4a16_gemm_ref(to_f32(x), oracle_packed(q.cpu(), s.cpu(), None if z is None else z.cpu(), 128),
                            to_f32(lin.bias.detach().half()))
    assert_close(y.cpu(), ref, "float16", what="from_dense w4a16")


@pytest.mark.parametrize("m", [1, 64, 300])
def test_fp8_module_forward_matches_oracle(m):
    n, k = 768, 1024
    lin = torch.nn.Linear(k, n)
    with torch.no_grad():
        lin.weight.mul_(0.5)
    mod = ops.make_packed_linear("fp8", lin.to(DEV), granularity="per_channel")
    w = lin.weight.detach().cpu().numpy()
    wq, sw = og.quantize_fp8_ref(w, "per_channel")
    assert np.array_equal(fp8_codes(mod.weight_fp8), wq)
    assert np.array_equal(mod.weight_scale.cpu().numpy().reshape(-1), sw.reshape(-1))
    x = x_act(m, k, torch.bfloat16, seed=m)
    y = mod(x.to(DEV))
    assert ops.last_path("fp8_linear") == "hip" and y.dtype == torch.bfloat16
    xq, sx = og.quantize_fp8_ref(to_f32(x), "per_token")
    bias = to_f32(lin.bias.detach().cpu().bfloat16())
    ref = og.fp8_gemm_ref(xq, sx, wq, sw, bias)
    assert_close(y.cpu(), ref, "bfloat16", what=f"KernelFp8Linear m={m}")
    fresh = ops.make_packed_linear("fp8", in_features=k, out_features=n, bias=torch.zeros(n), device=DEV)
    fresh.load_state_dict(mod.state_dict())
    assert torch.equal(fresh(x.to(DEV)), y)


@pytest.mark.parametrize("m", [1, 64, 300])
def test_int8_module_forward_is_exact(m):
    n, k = 640, 2048
    lin = torch.nn.Linear(k, n)
    mod = ops.make_packed_linear("int8", lin.to(DEV))
    w = lin.weight.detach().cpu().numpy()
    wq, sw = og.quantize_int8_ref(w, "per_channel")
    assert np.array_equal(mod.weight_int8.cpu().numpy(), wq)
    assert np.array_equal(mod.weight_scale.cpu().numpy(), sw.reshape(-1))
    x = x_act(m, k, torch.bfloat16, seed=m + 7)
    y = mod(x.to(DEV))
    assert ops.last_path("int8_linear") == "hip" and y.dtype == torch.bfloat16
    xq, sx = og.quantize_int8_ref(to_f32(x), "per_token")
    bias = to_f32(lin.bias.detach().cpu().bfloat16())
    ref = og.int8_gemm_ref(xq, sx, wq, sw, bias)
    assert torch.equal(y.cpu(), torch.from_numpy(ref).to(torch.bfloat16))
    fresh = ops.make_packed_linear("int8", in_features=k, out_features=n, bias=torch.zeros(n), device=DEV)
    fresh.load_state_dict(mod.state_dict())
    assert torch.equal(fresh(x.to(DEV)), y)


@pytest.mark.parametrize("kind,kw", [("fp8", {"granularity": "per_channel"}), ("fp8", {"granularity": "per_tensor"}),
                                     ("fp8", {"granularity": "block2d", "block": 128}), ("int8", {})])
def test_w8a8_module_quantised_on_host_then_moved(kind, kw):
    """A checkpoint quantised on the CPU, then moved to the GPU (the reference's flow): its codes and scales equal
    the device quantisers' bit for bit, and its forward matches the same module built on the GPU bit for bit."""
    n, k = 384, 1024
    lin = torch.nn.Linear(k, n)
    with torch.no_grad():
        lin.weight.mul_(0.5)
        lin.weight[5] = 0.0
    host = ops.make_packed_linear(kind, lin, **kw)
    assert all(not t.is_cuda for t in host.state_dict().values())
    moved = host.to(DEV)
    dev_mod = ops.make_packed_linear(kind, torch.nn.Linear(k, n).to(DEV).requires_grad_(False), **kw)
    with torch.no_grad():
        dev_mod.weight_scale.zero_()
        dev_mod.bias.copy_(lin.bias.detach().to(DEV))
    if kind == "fp8":
        qd, sd = ops.quantize_weight_fp8(lin.weight.detach().to(DEV), kw["granularity"], kw.get("block", 128))
        assert torch.equal(moved.weight_fp8.view(torch.uint8), qd.view(torch.uint8))
        assert torch.equal(moved.weight_scale, sd.reshape(moved.weight_scale.shape))
        with torch.no_grad():
            dev_mod.weight_fp8.copy_(qd)
            dev_mod.weight_scale.copy_(sd.reshape(dev_mod.weight_scale.shape))
    else:
        qd, sd = ops.quantize_weight_int8(lin.weight.detach().to(DEV))
        assert torch.equal(moved.weight_int8, qd) and torch.equal(moved.weight_scale, sd)
        with torch.no_grad():
            dev_mod.weight_int8.copy_(qd)
            dev_mod.weight_scale.copy_(sd)
    x = x_act(33, k, torch.bfloat16, seed=9).to(DEV)
    y = moved(x)
    assert torch.equal(y, dev_mod(x))
    assert ops.last_path(f"{kind}_linear") == "hip"
    fresh = ops.make_packed_linear(kind, in_features=k, out_features=n, bias=torch.zeros(n), device=DEV, **kw)
    fresh.load_state_dict(host.state_dict())
    assert torch.equal(fresh(x), y)


@pytest.mark.parametrize("m", [1, 16, 64])
def test_w4a16_module_keeps_a_cdna4_copy_for_decode_rows(m, monkeypatch):
    """A portable_row module on the GPU keeps a CDNA4-layout copy and serves 3..64-row calls from it (one row stays on
    the split-K GEMV); its state dict stays portable_row; the copy follows a state-dict load; FORGE_W4_CDNA4_COPY=0
    keeps every call on portable_row.  Each path against the oracle."""
    n, k, gs = 1536, 2048, 128
    q, s, z = w4_parts(n, k, gs, False, seed=m + 40)
    mod = ops.KernelW4A16Linear.from_packed(L.pack_w4(q, s, z, gs).to(DEV))
    x = x_act(m, k, torch.bfloat16, seed=m + 41).to(DEV)
    ref = og.w4a16_gemm_ref(to_f32(x.cpu()), oracle_packed(q, s, z, gs))
    y = mod(x)
    kern = ops.last_kernel()
    assert ("cdna4" in kern or "w4_frag_kernel" in kern) == (m > 1), kern
    assert_close(y.cpu(), ref, "bfloat16", what=f"module with CDNA4 copy m={m}")
    sd = mod.state_dict()
    assert sd["qweight"].shape == L.pack_w4(q, s, z, gs).qweight.shape  # portable_row in the checkpoint
    fresh = ops.make_packed_linear("w4a16", in_features=k, out_features=n, group_size=gs, sym=False,
                                   dtype=torch.float16, device=DEV)
    fresh.load_state_dict(sd)
    assert torch.equal(fresh(x), y), "the reloaded module's copy does not match"
    monkeypatch.setenv("FORGE_W4_CDNA4_COPY", "0")
    plain = ops.KernelW4A16Linear.from_packed(L.pack_w4(q, s, z, gs).to(DEV))
    yp = plain(x)
    assert "w4_frag_kernel" not in ops.last_kernel() and "cdna4" not in ops.last_kernel()
    assert_close(yp.cpu(), ref, "bfloat16", what=f"module without copy m={m}")
