"""CPU tests of the C ABI: the library loads, exports every symbol include/forge_mi355x.h declares, and its
argument validation rejects bad calls before touching the GPU (no kernel is launched here)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from forge_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "forge_mi355x.h")


def declared_symbols() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fg_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    syms = declared_symbols()
    for s in ("fg_w4a16_gemm", "fg_w4a16_workspace_bytes", "fg_w4_dequant", "fg_int8_gemm", "fg_fp8_gemm",
              "fg_quant_int8_rowwise", "fg_quant_fp8_rowwise", "fg_quant_fp8_block", "fg_version", "fg_last_error",
              "fg_device_ok", "fg_last_kernel"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    assert set(_lib.SIGNATURES) == set(declared_symbols())


def test_version_and_error_reporting_without_gpu():
    L = _lib.lib()
    assert L.fg_version().decode().startswith("forge_mi355x")
    rc = L.fg_w4a16_gemm(None, 0, 2, None, 0, None, 1, 0, None, 0, None, None, None, 0, None, 0, -1, 4, 4, 128, 1,
                         None, None, 0, None)
    assert rc == _lib.EINVAL and "bad sizes" in _lib.last_error()
    rc = L.fg_int8_gemm(None, 0, None, 0, None, 0, None, 0, None, 0, None, 0, 0, 4, 4, 4, None, None)
    assert rc == _lib.EINVAL and "null tensor" in _lib.last_error()
    rc = L.fg_fp8_gemm(None, 0, None, 0, 0, None, 0, None, 0, 0, 1, 1, 128, None, 0, None, 0, 0, 0, 4, 4, None, None)
    assert rc == _lib.OK  # M == 0 is a no-op
    rc = L.fg_quant_fp8_block(None, 0, 2, None, 0, None, 0, 4, 4, 0, 128, None, None)
    assert rc == _lib.EINVAL


def test_mm_config_and_int32_bias_are_validated_before_launch():
    """Host-side rejections (the pointers are placeholders that no kernel ever sees)."""
    L = _lib.lib()
    dummy = ctypes.c_void_p(256)
    rc = L.fg_int8_gemm(dummy, 128, None, 0, dummy, 128, None, 0, dummy, _lib.F32, dummy, 64, _lib.I32, 64, 64, 128,
                        None, None)
    assert rc == _lib.EINVAL and "bias" in _lib.last_error()
    for t in (32, 512, 1):
        cfg = _lib.MMConfig(t, 0)
        rc = L.fg_int8_gemm(dummy, 128, None, 0, dummy, 128, None, 0, None, 0, dummy, 64, _lib.I32, 64, 64, 128,
                            ctypes.byref(cfg), None)
        # tile_m = 1 is the INT8 decode GEMV, which 64 rows cannot take
        assert rc == (_lib.EUNSUPPORTED if t == 1 else _lib.EINVAL) and "tile_m" in _lib.last_error(), t
        rc = L.fg_fp8_gemm(dummy, 128, dummy, 1, 0, dummy, 128, dummy, 1, 0, 1, 1, 128, None, 0, dummy, 64, _lib.BF16,
                           64, 64, 128, ctypes.byref(cfg), None)
        assert rc == _lib.EINVAL and "tile_m" in _lib.last_error(), t


@pytest.mark.parametrize("m,n,k,expect_ws", [(1, 4096, 4096, False), (4, 4096, 4096, False), (16, 4096, 4096, True),
                                            (512, 4096, 4096, True), (768, 4096, 28672, True), (768, 28672, 4096, False),
                                            (4096, 4096, 4096, False)])
def test_workspace_query_follows_the_kernel_plan(m, n, k, expect_ws):
    """Split-K partials only (no kernel keeps a dequantised copy of the weights): none once the tiles cover the CUs."""
    L = _lib.lib()
    ws = L.fg_w4a16_workspace_bytes(m, n, k, 128, 1, 1, 0, None)
    assert (ws > 0) == expect_ws
    if ws:
        assert ws % (m * n * 4) == 0 and ws // (m * n * 4) > 1
    # FG_W4_DEQUANT_GEMM (the reference's dequant_matmul) names the prefill kernels: their workspace
    dq = _lib.W4Config(_lib.W4_DEQUANT_GEMM, 0, 0, 0, 0)
    pf = _lib.W4Config(_lib.W4_PREFILL, 0, 0, 0, 0)
    assert L.fg_w4a16_workspace_bytes(m, n, k, 128, 1, 1, 0, ctypes.byref(dq)) == \
        L.fg_w4a16_workspace_bytes(m, n, k, 128, 1, 1, 0, ctypes.byref(pf))
    # forcing one split removes the workspace
    cfg = _lib.W4Config(_lib.W4_MFMA, 0, 0, 0, 1)
    assert L.fg_w4a16_workspace_bytes(m, n, k, 128, 1, 1, 0, ctypes.byref(cfg)) == 0
    # a g_idx call goes to the generic kernel, which never needs one
    assert L.fg_w4a16_workspace_bytes(m, n, k, 128, 1, 1, 1, None) == 0


@pytest.mark.parametrize("m", [512, 768, 4096])
def test_w8a16_workspace_holds_split_partials_only(m):
    """The W8A16 prefill kernels' split-K partials (none once the tiles cover the CUs); FG_W4_DEQUANT_GEMM names them."""
    L = _lib.lib()
    n, k = 4096, 4096
    ws = L.fg_w8a16_workspace_bytes(m, n, k, -1, None)
    assert ws == 0 or (ws % (m * n * 4) == 0 and ws // (m * n * 4) > 1)
    assert (ws > 0) == (m < 4096)  # 256 tiles of 256 x 256 at 4096 rows cover the CUs in one pass
    dq = _lib.W4Config(_lib.W4_DEQUANT_GEMM, 0, 0, 0, 0)
    pf = _lib.W4Config(_lib.W4_PREFILL, 0, 0, 0, 0)
    assert L.fg_w8a16_workspace_bytes(m, n, k, -1, ctypes.byref(dq)) == L.fg_w8a16_workspace_bytes(m, n, k, -1,
                                                                                                    ctypes.byref(pf))


def _header_prototypes() -> dict[str, list[str]]:
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    protos = {}
    for m in re.finditer(r"\b(fg_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = [a.strip() for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        protos[m.group(1)] = params
    return protos


def _ctype_for(param: str):
    t = param.rsplit(" ", 1)[0] if not param.endswith("*") else param
    if "*" in param:
        return ctypes.c_void_p if "fg_w4_config" not in param and "fg_mm_config" not in param else "struct*"
    t = t.replace("const ", "").strip()
    return {"int64_t": ctypes.c_int64, "int32_t": ctypes.c_int32, "int": ctypes.c_int, "size_t": ctypes.c_size_t,
            "float": ctypes.c_float, "fg_stream_t": ctypes.c_void_p}[t]


def test_ctypes_signatures_match_the_header_parameter_types():
    """A 64-bit parameter bound as a 32-bit ctypes int would leave garbage in the upper half of its register."""
    protos = _header_prototypes()
    assert set(protos) == set(_lib.SIGNATURES)
    for name, params in protos.items():
        args, _ = _lib.SIGNATURES[name]
        assert len(args) == len(params), name
        for a, p in zip(args, params):
            want = _ctype_for(p)
            if want == "struct*":
                assert getattr(a, "_type_", None) in (_lib.W4Config, _lib.MMConfig), (name, p)
            else:
                assert ctypes.sizeof(a) == ctypes.sizeof(want) and a in (want, ctypes.c_int32, ctypes.c_int), (name, p, a)
