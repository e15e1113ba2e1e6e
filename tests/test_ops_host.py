"""CPU tests of the host-side op layer: it refuses to compute off the GPU (no silent CPU fallback), validates input
like the reference dispatcher, and keeps the reference's module/state-dict surface."""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn

from forge_amd import _lib
from forge_amd import layouts as L
from forge_amd import ops_gemm as ops
from forge_amd.errors import ConfigError, HardwareUnsupported
from tests._util import w4_parts


def test_cpu_tensors_raise_instead_of_falling_back():
    q, s, z = w4_parts(48, 96, 32, False)
    p = L.pack_w4(q, s, z, 32)
    x = torch.randn(5, 96).bfloat16()
    with pytest.raises(HardwareUnsupported):
        ops.w4a16_linear(x, p)
    with pytest.raises(HardwareUnsupported):
        ops.quantize_act_int8(x.float())
    with pytest.raises(HardwareUnsupported):
        ops.quantize_act_fp8(x.float())
    with pytest.raises(HardwareUnsupported):
        ops.int8_linear(torch.zeros(2, 8, dtype=torch.int8), torch.zeros(4, 8, dtype=torch.int8), torch.ones(4),
                        x_scale=torch.ones(2))
    with pytest.raises(HardwareUnsupported):
        p.dequantize()
    assert ops.last_path("w4a16_linear") is None or ops.last_path("w4a16_linear") == "hip"


def test_force_ref_is_refused(monkeypatch):
    monkeypatch.setenv("FORGE_FORCE_REF", "1")
    assert ops.force_ref() and ops.kernel_strict()
    with pytest.raises(HardwareUnsupported, match="FORGE_FORCE_REF"):
        ops.quantize_act_int8(torch.zeros(1, 4))


def test_user_errors_are_config_errors():
    with pytest.raises(ConfigError):
        ops.fp8_linear(torch.zeros(2, 8, dtype=torch.float8_e4m3fn), torch.zeros(4, 8, dtype=torch.float8_e4m3fn),
                       torch.ones(4))  # pre-quantised without x_scale
    with pytest.raises(ConfigError):
        ops.int8_linear(torch.zeros(2, 8, dtype=torch.int8), torch.zeros(4, 8, dtype=torch.int8), torch.ones(4))
    assert issubclass(ConfigError, ValueError)


@pytest.mark.parametrize("sx_shape,sw_shape,mode", [((1,), (1,), 0), ((7,), (33,), 1), ((1,), (33,), 1),
                                                    ((7, 2), (33, 2), 2), ((7, 2), (1, 2), 2), ((7,), (1, 2), 2),
                                                    ((1,), (33,), 1)])
def test_prepare_fp8_scales_modes(sx_shape, sw_shape, mode):
    """Every granularity mix normalises to in-bounds element strides (tests/test_kernels_gemm_review.py:94-106)."""
    m, n, k, block = 7, 33, 200, 128
    got = ops.prepare_fp8_scales(torch.ones(sx_shape), torch.ones(sw_shape), m, n, k, block)
    assert got[0] == mode
    sam, sak, sbn, sbk = got[3]
    sa, sb, div = got[1], got[2], got[4]
    kb = -(-k // block)
    assert (m - 1) * sam + (kb - 1) * sak < sa.numel() and ((n - 1) // div) * sbn + (kb - 1) * sbk < sb.numel()


def test_prepare_fp8_scales_rejects_mismatches():
    with pytest.raises(ValueError):
        ops.prepare_fp8_scales(torch.ones(3), torch.ones(33), 7, 33, 200, 128)
    with pytest.raises(ValueError):
        ops.prepare_fp8_scales(torch.ones(7, 1), torch.ones(33, 2), 7, 33, 200, 128)


def test_w4_config_aliases(monkeypatch):
    assert ops._w4_config(None) is None
    assert ops._w4_config({"impl": "dot"}).impl == 2 and ops._w4_config({"impl": "legacy"}).impl == 3
    assert ops._w4_config({"impl": "prefill"}).impl == 4
    assert ops._w4_config({"impl": "gemv", "rows_per_wave": 2}).rows_per_wave == 2
    assert ops._w4_config({"impl": "gemv", "gemv_kernel": "tile"}).gemv_kernel == 2
    assert ops._w4_config({"impl": "gemv"}).gemv_kernel == 0
    with pytest.raises(ConfigError):
        ops._w4_config({"impl": "gemv", "gemv_kernel": "lds"})
    with pytest.raises(ConfigError):
        ops._w4_config({"impl": "bogus"})
    monkeypatch.setenv("FORGE_W4_IMPL", "dequant_matmul")
    assert ops._w4_config(None).impl == _lib.W4_DEQUANT_GEMM
    monkeypatch.setenv("FORGE_W4_IMPL", "dot")
    assert ops._w4_config(None).impl == _lib.W4_MFMA


def test_packed_linear_modules_keep_reference_buffer_names():
    m = ops.make_packed_linear("w4a16", in_features=96, out_features=40, bias=torch.zeros(40), group_size=32, sym=False)
    assert set(m.state_dict()) == {"bias", "qweight", "scales", "zeros"}
    assert m.qweight.shape == (40, 12) and m.scales.shape == (3, 40) and m.zeros.shape == (3, 5)
    f = ops.make_packed_linear("fp8", in_features=96, out_features=40, granularity="block2d", block=32)
    assert set(f.state_dict()) == {"weight_fp8", "weight_scale"} and f.weight_scale.shape == (2, 3)
    i = ops.make_packed_linear("int8", in_features=96, out_features=40)
    assert set(i.state_dict()) == {"weight_int8", "weight_scale"}
    with pytest.raises(ConfigError):
        ops.make_packed_linear("nvfp4", in_features=4, out_features=4)
    # dense -> W4 packing is a load-time data op and works anywhere; the module round-trips its state dict
    lin = nn.Linear(96, 40)
    w4 = ops.make_packed_linear("w4a16", lin, group_size=32)
    fresh = ops.make_packed_linear("w4a16", in_features=96, out_features=40, bias=lin.bias, group_size=32)
    fresh.load_state_dict(w4.state_dict())
    assert torch.equal(fresh.qweight, w4.qweight) and torch.equal(fresh.scales, w4.scales)


def test_w8_packer_matches_oracle_and_module_surface():
    """PackedW8 (forge/kernels/layouts/w8.py:18-104): same bytes as the oracle packer, exact dequantisation, the
    reference's RTN (scale = amax / 127 rounded to fp16, q clamped to [-128, 127]) and the module's buffer names."""
    import numpy as np

    from oracle import gemm as og

    g = torch.Generator().manual_seed(3)
    w = torch.randn(40, 96, generator=g)
    q, s = L.quantize_w8_rtn(w, 32)
    assert q.dtype == torch.int8 and s.dtype == torch.float16 and s.shape == (40, 3)
    amax = w.view(40, 3, 32).abs().amax(-1)
    assert torch.equal(s, (amax / 127.0).clamp_min(1e-12).to(torch.float16))
    assert (w.view(40, 3, 32) / s.float().unsqueeze(-1) - q.view(40, 3, 32).float()).abs().max() <= 0.5 + 1e-4
    p = L.pack_w8(q, s, 32)
    op = og.pack_w8(q.numpy(), s.float().numpy(), 32)
    assert np.array_equal(p.qweight.numpy(), op["qweight"]) and np.array_equal(p.scales.float().numpy(), op["scales"])
    assert np.array_equal(p.dequantize().numpy(), og.dequantize_w8(op))
    assert p.layout_id == "w8.portable_row.v1-db2653" and p.num_groups == 3
    q2, s2 = L.unpack_w8(p)
    assert torch.equal(q2, q) and torch.equal(s2, s)
    m = ops.make_packed_linear("w8a16", packed=p, bias=torch.zeros(40))
    assert set(m.state_dict()) == {"bias", "qweight", "scales"} and m.scales.shape == (3, 40)
    assert m.quant_spec() == {"bits": 8, "group_size": 32, "layout": "w8.portable_row.v1-db2653"}
    with pytest.raises(ConfigError):
        L.pack_w8(q, s[:, :2], 32)
    with pytest.raises(ConfigError):
        ops.make_packed_linear("w4a16", packed=p)
