"""GEMM-family dispatchers and packed-linear modules, backed only by libforge_mi355x.so (hand-written gfx950 HIP).

Drop-in mirror of the reference's ``forge/kernels/ops_gemm.py`` (signatures of ``w4a16_linear`` :287-317,
``fp8_linear`` :396-461, ``int8_linear`` :483-515, ``quantize_act_fp8`` :359-388, ``quantize_act_int8`` :467-480,
``quantize_weight_fp8`` :391-393, ``prepare_w4`` :267-277, the ``Kernel*Linear`` modules :769-961 and
``make_packed_linear`` :1025-1068, with the same buffer names so state dicts load unchanged).

Differences from the reference, on purpose:

* There is exactly one path, the HIP library.  ``last_path(op)`` returns ``"hip"``.  A tensor that is not on a gfx950
  GPU, a missing library, ``FORGE_FORCE_REF=1`` or a kernel error raises instead of silently falling back to a torch
  oracle (the reference warns and serves its CPU oracle; ``FORGE_KERNEL_STRICT=1`` is therefore always in effect).
* Every launch is host-sync free and allocates only through torch's caching allocator on the current stream (outputs
  and the split-K workspace), so calls can be captured in a HIP graph.
"""
from __future__ import annotations

import logging
import os
import threading
from typing import Any, ClassVar

import torch
import torch.nn as nn

from . import _lib
from .errors import ConfigError, HardwareUnsupported
from .layouts import (
    KIND_PORTABLE,
    MISSING_SORT,
    PORTABLE_W4,
    PORTABLE_W8,
    Layout,
    PackedW4,
    PackedW8,
    cached_group_sort,
    effective_group,
    get_layout,
    num_groups,
    pack_w4,
    pack_w8,
    quantize_w4_rtn,
    quantize_w8_rtn,
    repack,
    roundup,
)

log = logging.getLogger("forge_amd.ops_gemm")

_LAST_PATH: dict[str, str] = {}
_WARNED: set[str] = set()
_LOCK = threading.Lock()
FP8_E4M3_MAX = 448.0


# ------------------------------------------------------------------------------------------------ environment
def force_ref() -> bool:
    return os.environ.get("FORGE_FORCE_REF", "0") == "1"


def kernel_debug() -> bool:
    return os.environ.get("FORGE_KERNEL_DEBUG", "0") == "1"


def kernel_strict() -> bool:
    """Always true in this build: kernel failures raise (there is no fallback path to serve the call)."""
    return True


def last_path(op: str) -> str | None:
    """Path taken by the last call of ``op`` (``"hip"`` for every op of this build)."""
    return _LAST_PATH.get(op)


def reset_failure_memo() -> None:
    """Kept for API compatibility: this build memoises no failures (nothing falls back)."""


def _note(op: str, path: str = "hip", why: str = "") -> None:
    _LAST_PATH[op] = path
    if kernel_debug():
        log.info("%s -> %s%s", op, path, f" ({why})" if why else "")


def _warn_once(key: str, msg: str) -> None:
    with _LOCK:
        if key in _WARNED:
            return
        _WARNED.add(key)
    log.warning(msg)


def _ready(t: torch.Tensor, op: str) -> None:
    if force_ref():
        raise HardwareUnsupported(f"{op}: FORGE_FORCE_REF=1 requests the torch reference path, which is not part of "
                                  "forge_amd (run the reference implementation for that)")
    _lib.require_device(t, op)


def _capturing(t: torch.Tensor) -> bool:
    try:
        return bool(t.is_cuda and torch.cuda.is_current_stream_capturing())
    except Exception:  # noqa: BLE001
        return False


def _rows(x: torch.Tensor) -> torch.Tensor:
    """``x [..., K]`` as a 2-D ``[M, K]`` view with unit stride along K (copy only when needed)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < x2.shape[1]):
        x2 = x2.contiguous()
    return x2


def _ld(t: torch.Tensor) -> int:
    """Row stride for the C ABI: the dim-0 stride, or the row length for a one-row tensor (torch counts a one-row
    tensor contiguous whatever its dim-0 stride is, so that stride can be smaller than a row)."""
    return int(t.stride(0)) if t.shape[0] > 1 else int(t.shape[1])


# ------------------------------------------------------------------------------------------------ W4A16
def _data_stamp(*ts: torch.Tensor | None) -> tuple:
    return tuple((t.data_ptr(), t._version, tuple(t.shape), str(t.device)) for t in ts if t is not None)


def _portable(packed: PackedW4) -> PackedW4:
    """``packed`` in portable_row (a fragment-layout artifact is repacked once, cache stamped by tensor identity)."""
    if packed.layout.kind == KIND_PORTABLE:
        return packed
    stamp = _data_stamp(packed.qweight, packed.scales, packed.zeros, packed.g_idx)
    cache = packed.meta.setdefault("_repack_cache", {})
    hit = cache.get(PORTABLE_W4.id)
    if hit is None or hit[0] != stamp:
        hit = cache[PORTABLE_W4.id] = (stamp, repack(packed, PORTABLE_W4))
    return hit[1]


def prepare_w4(packed: PackedW4) -> PackedW4:
    """Precompute launch metadata (portable repack, act-order column sort) so that ``w4a16_linear`` never syncs;
    call after packing / loading / moving a weight, outside graph capture.  Returns the portable weight."""
    p = _portable(packed)
    if p.g_idx is not None:
        cached_group_sort(p, compute=True)
    return p


_IMPL_ALIASES = {"gemv": "gemv", "dot": "mfma", "mfma": "mfma", "dequant_matmul": "mfma", "prefill": "prefill",
                 "legacy": "generic", "generic": "generic", "auto": None, None: None}


def forced_impl() -> str | None:
    """``FORGE_W4_IMPL`` = gemv | mfma | prefill | generic (reference names dot / dequant_matmul / legacy are accepted)."""
    v = os.environ.get("FORGE_W4_IMPL", "").strip().lower()
    return _IMPL_ALIASES.get(v) if v in _IMPL_ALIASES else None


def _w4_config(config: dict[str, Any] | None) -> _lib.W4Config | None:
    impl = forced_impl() or _IMPL_ALIASES.get((config or {}).get("impl"), None)
    if not config and impl is None:
        return None
    c = config or {}
    if c.get("impl") not in _IMPL_ALIASES:
        raise ConfigError(f"unknown W4A16 impl {c.get('impl')!r}; choose gemv, mfma, prefill or generic")
    if c.get("gemv_kernel") not in _lib.GEMV_KERNEL:
        raise ConfigError(f"unknown GEMV kernel {c.get('gemv_kernel')!r}; choose split, tile or wave")
    return _lib.W4Config(_lib.W4_IMPL[impl], int(c.get("rows_per_wave") or 0), int(c.get("max_blocks") or 0),
                         int(c.get("tile_m") or 0), int(c.get("split_k") or 0), int(c.get("tile_n") or 0),
                         _lib.GEMV_KERNEL[c.get("gemv_kernel")])


def _w4_launch(x2: torch.Tensor, p: PackedW4, perm: torch.Tensor | None, g_idx: torch.Tensor | None,
               bias: torch.Tensor | None, y: torch.Tensor, cfg: _lib.W4Config | None) -> None:
    L = _lib.lib()
    m, k = x2.shape
    n = p.n
    gs = p.group_size
    x_aligned = int(_ld(x2) % 8 == 0 and x2.data_ptr() % 16 == 0)
    q_aligned = int(_ld(p.qweight) % 4 == 0 and p.qweight.data_ptr() % 16 == 0)
    cfgp = None if cfg is None else _lib.ctypes.byref(cfg)
    ws_bytes = L.fg_w4a16_workspace_bytes(m, n, k, gs, x_aligned, q_aligned, int(g_idx is not None), cfgp)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x2.device) if ws_bytes else None
    zeros = p.zeros
    _lib.check(L.fg_w4a16_gemm(
        _lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(p.qweight), _ld(p.qweight),
        _lib.ptr(p.scales), _lib.dtype_code(p.scales.dtype), _ld(p.scales),
        _lib.ptr(zeros), 0 if zeros is None else _ld(zeros), _lib.ptr(perm), _lib.ptr(g_idx),
        _lib.ptr(bias), _lib.dtype_code(bias.dtype) if bias is not None else 0,
        _lib.ptr(y), y.stride(0), m, n, k, gs, p.num_groups, cfgp, _lib.ptr(ws), ws_bytes, _lib.stream_of(x2)),
        "fg_w4a16_gemm")


def w4a16_linear(x: torch.Tensor, packed: PackedW4, bias: torch.Tensor | None = None, *,
                 config: dict[str, Any] | None = None, deterministic: bool = True) -> torch.Tensor:
    """``y = x @ dequant(W)^T + bias`` for ``x [..., K]`` bf16/fp16 on a gfx950 GPU (returns ``x.dtype``).

    Kernel by the C library's policy (override with ``config={"impl": "gemv"|"mfma"|"generic", ...}`` or
    ``FORGE_W4_IMPL``): for M <= 4 a GEMV (``gemv_kernel``: "split" = register-resident split-K kernel, "tile" =
    LDS-tiled kernel, "wave" = one wavefront per row block; chosen per shape and operand alignment), dequantise-to-LDS
    + bf16/fp16 MFMA otherwise, and a per-element generic kernel for irregular act-order or unaligned weights.  All paths reduce in a fixed order
    (``deterministic`` is accepted for API compatibility; results are always run-to-run reproducible).
    """
    _ready(x, "w4a16_linear")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise HardwareUnsupported(f"w4a16_linear: activations must be bf16 or fp16, got {x.dtype}")
    if x.shape[-1] != packed.k:
        raise ConfigError(f"x has K={x.shape[-1]} but the packed weight has K={packed.k}")
    p = _portable(packed)
    if p.qweight.device != x.device:
        raise ConfigError(f"weight on {p.qweight.device} but x on {x.device}")
    lead = x.shape[:-1]
    x2 = _rows(x)
    m = x2.shape[0]
    y = torch.empty((m, p.n), dtype=x.dtype, device=x.device)
    if m == 0:
        _note("w4a16_linear")
        return y.reshape(*lead, p.n)
    w, perm, g_idx = p, None, None
    if p.g_idx is not None:
        srt = cached_group_sort(p, compute=not _capturing(x2))
        if srt is MISSING_SORT:
            _warn_once("w4_capture", "act-order W4 weight not prepared before graph capture (call prepare_w4): "
                                     "using the per-column g_idx kernel")
            g_idx = p.g_idx
        elif srt is None:
            g_idx = p.g_idx
        else:
            w, perm = srt
    b = None if bias is None else bias.contiguous()
    _w4_launch(x2, w, perm, g_idx, b, y, _w4_config(config))
    _note("w4a16_linear")
    return y.reshape(*lead, p.n)


# ------------------------------------------------------------------------------------------------ W8A16
def w8a16_linear(x: torch.Tensor, packed: PackedW8, bias: torch.Tensor | None = None, *,
                 config: dict[str, Any] | None = None, deterministic: bool = True) -> torch.Tensor:
    """``y = x @ dequant(Wq)^T + bias`` with symmetric int8 weights (``forge/kernels/ops_gemm.py:320-346``) for
    ``x [..., K]`` bf16/fp16 on a gfx950 GPU (returns ``x.dtype``).

    ``fg_w8a16_gemm`` picks the skinny MFMA kernel for M <= 64, the dequantise-to-LDS MFMA kernel beyond, and a
    generic kernel for shapes neither takes (override with ``config={"impl": "mfma"|"prefill"|"generic"}``).  Every
    path reduces in a fixed order, so results are run-to-run reproducible.
    """
    _ready(x, "w8a16_linear")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise HardwareUnsupported(f"w8a16_linear: activations must be bf16 or fp16, got {x.dtype}")
    if x.shape[-1] != packed.k:
        raise ConfigError(f"x has K={x.shape[-1]} but the packed weight has K={packed.k}")
    if packed.layout.bits != 8:
        raise ConfigError(f"layout {packed.layout_id} is not an 8-bit layout")
    if packed.qweight.device != x.device:
        raise ConfigError(f"weight on {packed.qweight.device} but x on {x.device}")
    lead = x.shape[:-1]
    x2 = _rows(x)
    m = x2.shape[0]
    y = torch.empty((m, packed.n), dtype=x.dtype, device=x.device)
    if m == 0:
        _note("w8a16_linear")
        return y.reshape(*lead, packed.n)
    q = packed.qweight if packed.qweight.stride(-1) == 1 else packed.qweight.contiguous()
    sc = packed.scales if packed.scales.stride(-1) == 1 else packed.scales.contiguous()
    b = None if bias is None else bias.contiguous()
    cfg = _w4_config(config)
    cfgp = None if cfg is None else _lib.ctypes.byref(cfg)
    L = _lib.lib()
    ws_bytes = L.fg_w8a16_workspace_bytes(m, packed.n, packed.k, packed.group_size, cfgp)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    _lib.check(L.fg_w8a16_gemm(
        _lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(q), _ld(q), _lib.ptr(sc),
        _lib.dtype_code(sc.dtype), _ld(sc), _lib.ptr(b),
        _lib.dtype_code(b.dtype) if b is not None else 0,
        _lib.ptr(y), y.stride(0), m, packed.n, packed.k, packed.group_size, packed.num_groups, cfgp, _lib.ptr(ws),
        ws_bytes, _lib.stream_of(x2)), "fg_w8a16_gemm")
    _note("w8a16_linear")
    return y.reshape(*lead, packed.n)


def w4_dequant(packed: PackedW4, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Dense ``[N, K]`` dequantisation on the GPU (``fg_w4_dequant``): ``(q - z) * s`` in fp32, one rounding."""
    p = _portable(packed)
    _ready(p.qweight, "w4_dequant")
    if dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ConfigError(f"w4_dequant: unsupported output dtype {dtype}")
    out = torch.empty((p.n, p.k), dtype=dtype, device=p.qweight.device)
    z = p.zeros
    L = _lib.lib()
    _lib.check(L.fg_w4_dequant(_lib.ptr(p.qweight), _ld(p.qweight), _lib.ptr(p.scales),
                               _lib.dtype_code(p.scales.dtype), _ld(p.scales), _lib.ptr(z),
                               0 if z is None else _ld(z), _lib.ptr(p.g_idx), _lib.ptr(out), _lib.dtype_code(dtype),
                               out.stride(0), p.n, p.k, p.group_size, p.num_groups, _lib.stream_of(out)),
               "fg_w4_dequant")
    _note("w4_dequant")
    return out


# ------------------------------------------------------------------------------------------------ FP8
def _flat_scale(s: torch.Tensor, rows: int | None = None) -> torch.Tensor:
    s = s.float()
    if s.dim() == 2 and s.numel() > 1 and ((rows is not None and s.shape in ((rows, 1), (1, rows)))
                                           or (rows is None and s.shape[1] == 1)):
        return s.reshape(-1)
    return s


def _quant_fp8_block(x2: torch.Tensor, bm: int, bk: int, scale: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor]:
    m, k = x2.shape
    q = torch.empty((m, k), dtype=torch.float8_e4m3fn, device=x2.device)
    nb, kb = -(-m // bm) if m else 0, -(-k // bk)
    if scale is not None:
        s = scale.float().reshape(1).to(x2.device).contiguous()
        static, out_s = s, None
    else:
        s = torch.empty((nb, kb), dtype=torch.float32, device=x2.device)
        static, out_s = None, s
    if m:
        _lib.check(_lib.lib().fg_quant_fp8_block(
            _lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(q), _ld(q), _lib.ptr(out_s),
            kb, m, k, bm, bk, _lib.ptr(static), _lib.stream_of(x2)), "fg_quant_fp8_block")
    return q, s


def quantize_act_fp8(x: torch.Tensor, *, granularity: str = "per_token", block: int = 128,
                     scale: torch.Tensor | None = None, rms_weight: torch.Tensor | None = None,
                     rms_eps: float | None = None, fmt: str = "e4m3") -> tuple[torch.Tensor, torch.Tensor]:
    """Dynamic (or static ``scale=``) FP8 e4m3fn quantisation of ``x [..., K]`` -> ``(q, scale fp32)``.

    Scale shapes follow the reference oracle: per_token ``[M]``, per_tensor ``[1]``, block ``[M, ceil(K/block)]``,
    block2d ``[ceil(M/block), ceil(K/block)]``.  ``rms_eps`` fuses RMSNorm (times ``rms_weight``) in front of the
    per-token absmax.
    """
    _ready(x, "quantize_act_fp8")
    if fmt != "e4m3":
        raise HardwareUnsupported("quantize_act_fp8: only OCP e4m3fn is supported on gfx950 in this build")
    if not x.is_floating_point():
        raise ConfigError("quantize_act_fp8: x must be a float tensor")
    shape = x.shape
    x2 = _rows(x)
    m, k = x2.shape
    g = "per_token" if granularity == "per_channel" else granularity
    if rms_eps is not None and g != "per_token":
        raise ConfigError("fused RMSNorm requires per-token granularity")
    L = _lib.lib()
    if g == "per_token":
        q = torch.empty((m, k), dtype=torch.float8_e4m3fn, device=x.device)
        s = torch.empty(m, dtype=torch.float32, device=x.device)
        st = None
        if scale is not None:
            st = scale.float().reshape(-1).to(x.device)
            if st.numel() == 1 and m != 1:
                st = st.expand(m)
            if st.numel() != m:
                raise ConfigError(f"static per-token scale has {st.numel()} entries for M={m}")
            st = st.contiguous()
            s = st
        w = None if rms_weight is None else rms_weight.contiguous()
        if m:
            _lib.check(L.fg_quant_fp8_rowwise(
                _lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(q), _ld(q),
                _lib.ptr(None if st is not None else s), m, k, _lib.ptr(st), _lib.ptr(w),
                _lib.dtype_code(w.dtype) if w is not None else 0, float(rms_eps or 0.0), int(rms_eps is not None),
                _lib.stream_of(x2)), "fg_quant_fp8_rowwise")
    elif g == "per_tensor":
        q, s = _quant_fp8_block(x2, max(m, 1), k, scale)
        s = s.reshape(1)
    elif g == "block":
        q, s = _quant_fp8_block(x2, 1, block, None if scale is None else scale)
    elif g == "block2d":
        q, s = _quant_fp8_block(x2, block, block, None if scale is None else scale)
    else:
        raise ConfigError(f"unknown granularity {granularity!r}")
    _note("quantize_act_fp8")
    return q.reshape(shape), s


def quantize_weight_fp8(w: torch.Tensor, granularity: str = "per_channel", block: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """Offline weight quantisation on the GPU: per_tensor | per_channel | block2d -> ``(w_fp8 [N,K], scale)``."""
    return quantize_act_fp8(w, granularity=granularity, block=block)


def prepare_fp8_scales(sx: torch.Tensor, sw: torch.Tensor, m: int, n: int, k: int, block: int):
    """Normalise any scale combination to ``(mode, sa, sb, (sa_m, sa_k, sb_n, sb_k), sb_div)`` element strides
    (0 = broadcast) -- the same rules as ``forge/kernels/triton/gemm_fp8.py:151-191``; bad sizes raise ValueError."""
    sxf, swf = sx.float().contiguous(), sw.float().contiguous()
    kb = -(-k // block)
    if sxf.dim() <= 1 and swf.dim() <= 1:
        if sxf.numel() == 1 and swf.numel() == 1:
            return 0, sxf.reshape(1), swf.reshape(1), (0, 0, 0, 0), block
        if sxf.numel() not in (1, m) or swf.numel() not in (1, n):
            raise ValueError(f"scale sizes {sxf.numel()}/{swf.numel()} do not match M={m}/N={n}")
        return 1, sxf.reshape(-1), swf.reshape(-1), (0 if sxf.numel() == 1 else 1, 0, 0 if swf.numel() == 1 else 1, 0), block
    if sxf.dim() == 2:
        if sxf.shape[0] != m or sxf.shape[1] < kb:
            raise ValueError(f"2-D activation scale must be [M={m}, >= {kb}], got {tuple(sxf.shape)}")
        sa, sam, sak = sxf, sxf.stride(0), sxf.stride(1)
    elif sxf.numel() in (1, m):
        sa, sam, sak = sxf.reshape(-1), (0 if sxf.numel() == 1 else 1), 0
    else:
        raise ValueError(f"activation scale has {sxf.numel()} entries for M={m}")
    if swf.dim() == 2:
        if swf.shape[1] < kb:
            raise ValueError(f"2-D weight scale needs >= {kb} columns, got {tuple(swf.shape)}")
        if swf.shape[0] == n:
            sb_div = 1
        elif swf.shape[0] >= -(-n // block):
            sb_div = block
        else:
            raise ValueError(f"2-D weight scale has {swf.shape[0]} rows for N={n}, block={block}")
        sb, sbn, sbk = swf, swf.stride(0), swf.stride(1)
    elif swf.numel() in (1, n):
        sb, sbn, sbk, sb_div = swf.reshape(-1), (0 if swf.numel() == 1 else 1), 0, 1
    else:
        raise ValueError(f"weight scale has {swf.numel()} entries for N={n}")
    return 2, sa, sb, (sam, sak, sbn, sbk), sb_div


def _mm_config(config: dict[str, Any] | None) -> _lib.MMConfig | None:
    if not config:
        return None
    return _lib.MMConfig(int(config.get("tile_m") or 0), int(config.get("tile_n") or 0))


def fp8_linear(x: torch.Tensor, w_fp8: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None = None, *,
               x_scale: torch.Tensor | None = None, act_granularity: str | None = None, block: int = 128,
               out_dtype: torch.dtype | None = None, config: dict[str, Any] | None = None) -> torch.Tensor:
    """``y = dq(quant(x)) @ dq(w)^T + bias`` on gfx950 fp8 matrix cores (OCP e4m3fn, fp32 accumulation).

    ``x`` float (dynamically quantised per token, or 1x``block`` when ``w_scale`` is 2-D) or pre-quantised e4m3fn
    with ``x_scale``.  Output dtype: ``out_dtype`` or ``x.dtype`` (bf16 for pre-quantised input).
    """
    ws = _flat_scale(w_scale, w_fp8.shape[0])
    pre = x.dtype in (torch.float8_e4m3fn, torch.float8_e5m2)
    odt = out_dtype or (torch.bfloat16 if pre else x.dtype)
    if odt not in (torch.float16, torch.bfloat16, torch.float32):
        odt = torch.bfloat16
    gran = act_granularity or ("block" if ws.dim() == 2 else ("per_tensor" if ws.numel() == 1 and x_scale is not None
                                                              and x_scale.numel() == 1 else "per_token"))
    if pre:
        if x_scale is None:
            raise ConfigError("pre-quantised fp8 activations need x_scale")
        xq, sx = x, _flat_scale(x_scale)
    else:
        xq, sx = quantize_act_fp8(x, granularity=gran, block=block, scale=x_scale)
    _ready(xq, "fp8_linear")
    if xq.dtype != torch.float8_e4m3fn or w_fp8.dtype != torch.float8_e4m3fn:
        raise HardwareUnsupported("fp8_linear: gfx950 kernels take float8_e4m3fn operands (e5m2 is not supported)")
    lead = xq.shape[:-1]
    a = _rows(xq)
    m, k = a.shape
    n = w_fp8.shape[0]
    if w_fp8.shape[1] != k:
        raise ConfigError(f"x has K={k} but the weight has K={w_fp8.shape[1]}")
    y = torch.empty((m, n), dtype=odt, device=xq.device)
    if m == 0:
        _note("fp8_linear")
        return y.reshape(*lead, n)
    try:
        mode, sa, sb, (sam, sak, sbn, sbk), sb_div = prepare_fp8_scales(sx.to(a.device), ws.to(a.device), m, n, k, block)
    except ValueError as e:
        raise ConfigError(str(e)) from e
    wq = w_fp8 if w_fp8.stride(-1) == 1 else w_fp8.contiguous()
    b = None if bias is None else bias.contiguous()
    cfg = _mm_config(config)
    _lib.check(_lib.lib().fg_fp8_gemm(
        _lib.ptr(a), _ld(a), _lib.ptr(sa), sam, sak, _lib.ptr(wq), _ld(wq), _lib.ptr(sb), sbn, sbk, sb_div,
        mode, block, _lib.ptr(b), _lib.dtype_code(b.dtype) if b is not None else 0, _lib.ptr(y), y.stride(0),
        _lib.dtype_code(odt), m, n, k, None if cfg is None else _lib.ctypes.byref(cfg), _lib.stream_of(a)),
        "fg_fp8_gemm")
    _note("fp8_linear")
    return y.reshape(*lead, n)


# ------------------------------------------------------------------------------------------------ INT8
def quantize_act_int8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token symmetric int8 -> ``(q int8, scale fp32 [M])``; bit-exact with the CPU oracle (IEEE division,
    round-half-even)."""
    _ready(x, "quantize_act_int8")
    if not x.is_floating_point():
        raise ConfigError("quantize_act_int8: x must be a float tensor")
    shape = x.shape
    x2 = _rows(x)
    m, k = x2.shape
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty(m, dtype=torch.float32, device=x.device)
    if m:
        _lib.check(_lib.lib().fg_quant_int8_rowwise(_lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(q),
                                                    _ld(q), _lib.ptr(s), m, k, _lib.stream_of(x2)),
                   "fg_quant_int8_rowwise")
    _note("quantize_act_int8")
    return q.reshape(shape), s


def int8_gemm(xq: torch.Tensor, sx: torch.Tensor | None, wq: torch.Tensor, sw: torch.Tensor | None,
              bias: torch.Tensor | None = None, *, out_dtype: torch.dtype = torch.bfloat16,
              config: dict[str, Any] | None = None) -> torch.Tensor:
    """Launcher on pre-quantised operands (the reference's ``int8_gemm_triton``, gemm_int8.py:95-137).
    ``out_dtype=torch.int32`` returns the raw exact accumulator."""
    _ready(xq, "int8_gemm")
    lead = xq.shape[:-1]
    a = _rows(xq)
    w = wq.contiguous()
    m, k = a.shape
    n = w.shape[0]
    if w.shape[1] != k:
        raise ConfigError(f"x has K={k} but the weight has K={w.shape[1]}")
    y = torch.empty((m, n), dtype=out_dtype, device=xq.device)
    if m == 0:
        return y.reshape(*lead, n)
    if out_dtype == torch.int32:
        if bias is not None:
            raise ConfigError("int8_gemm: a bias cannot be added to the raw int32 accumulator (out_dtype=torch.int32)")
        sa = sb = None
        sal = sbl = 0
    else:
        sa, sb = sx.float().reshape(-1).contiguous(), sw.float().reshape(-1).contiguous()
        if sa.numel() not in (1, m) or sb.numel() not in (1, n):
            raise ConfigError(f"scale sizes {sa.numel()}/{sb.numel()} do not match M={m}/N={n}")
        sal, sbl = sa.numel(), sb.numel()
    b = None if bias is None else bias.contiguous()
    cfg = _mm_config(config)
    _lib.check(_lib.lib().fg_int8_gemm(
        _lib.ptr(a), _ld(a), _lib.ptr(sa), sal, _lib.ptr(w), _ld(w), _lib.ptr(sb), sbl, _lib.ptr(b),
        _lib.dtype_code(b.dtype) if b is not None else 0, _lib.ptr(y), y.stride(0), _lib.dtype_code(out_dtype),
        m, n, k, None if cfg is None else _lib.ctypes.byref(cfg), _lib.stream_of(a)), "fg_int8_gemm")
    return y.reshape(*lead, n)


def int8_linear(x: torch.Tensor, w_int8: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None = None, *,
                x_scale: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                config: dict[str, Any] | None = None) -> torch.Tensor:
    """SmoothQuant-style W8A8 on gfx950 int8 matrix cores: ``x`` float (quantised per token here) or int8 with
    ``x_scale``; exact int32 accumulation, fp32 epilogue ``(acc * sx) * sw + bias``."""
    pre = x.dtype == torch.int8
    odt = out_dtype or (torch.bfloat16 if pre else x.dtype)
    if pre:
        if x_scale is None:
            raise ConfigError("int8 activations need x_scale")
        xq, sx = x, x_scale.float()
    else:
        xq, sx = quantize_act_int8(x)
    sw = _flat_scale(w_scale, w_int8.shape[0])
    y = int8_gemm(xq, sx, w_int8, sw, bias, out_dtype=odt, config=config)
    _note("int8_linear")
    return y


# ------------------------------------------------------------------------------------------------ modules
class _KernelLinear(nn.Module):
    """Common plumbing of the kernel-backed packed linears (buffers + optional bias parameter)."""

    kind: ClassVar[str] = ""

    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                 device: Any = None):
        super().__init__()
        self.in_features, self.out_features = int(in_features), int(out_features)
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=dtype or torch.float32, device=device))
        else:
            self.register_parameter("bias", None)

    def _bias(self, x: torch.Tensor) -> torch.Tensor | None:
        return None if self.bias is None else self.bias.to(x.dtype)

    def quant_spec(self) -> dict[str, Any]:
        return {}

    def extra_repr(self) -> str:
        return f"kind={self.kind}, in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}"


def _w4_shapes(n: int, k: int, group_size: int, layout: Layout, has_zeros: bool, n_groups: int | None = None):
    g = n_groups if n_groups is not None else -(-k // effective_group(group_size, k))
    if layout.kind == KIND_PORTABLE:
        n_pad, qshape = n, (n, roundup(k, 8) // 8)
    else:
        n_pad = roundup(n, 64)
        qshape = (roundup(k, 16) // 16, n_pad * 2)
    out = {"qweight": qshape, "scales": (g, n_pad)}
    if has_zeros:
        out["zeros"] = (g, roundup(n_pad, 8) // 8)
    return out


def _w4_prepare_hook(module: Any, _incompatible: Any) -> None:
    module.prepare()


class KernelW4A16Linear(_KernelLinear):
    """4-bit weight-only linear backed by :func:`w4a16_linear` (buffers ``qweight/scales/zeros/g_idx``)."""

    kind: ClassVar[str] = "w4a16"

    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                 device: Any = None, *, group_size: int = 128, sym: bool = True, layout: str | Layout | None = None,
                 has_g_idx: bool = False, n_groups: int | None = None, **_: Any):
        super().__init__(in_features, out_features, bias, dtype, device)
        self.group_size, self.sym = int(group_size), bool(sym)
        self.layout = PORTABLE_W4 if layout is None else (get_layout(layout) if isinstance(layout, str) else layout)
        shapes = _w4_shapes(out_features, in_features, group_size, self.layout, not sym, n_groups)
        self.register_buffer("qweight", torch.zeros(shapes["qweight"], dtype=torch.int32, device=device))
        self.register_buffer("scales", torch.zeros(shapes["scales"], dtype=dtype or torch.float16, device=device))
        self.register_buffer("zeros", torch.zeros(shapes["zeros"], dtype=torch.int32, device=device) if not sym else None)
        self.register_buffer("g_idx", torch.zeros(in_features, dtype=torch.int32, device=device) if has_g_idx else None)
        self._packed_meta: dict[str, Any] = {}
        self.register_load_state_dict_post_hook(_w4_prepare_hook)

    @classmethod
    def from_packed(cls, packed: PackedW4, bias: torch.Tensor | None = None) -> KernelW4A16Linear:
        m = cls(packed.k, packed.n, bias is not None, packed.scales.dtype, packed.qweight.device,
                group_size=packed.group_size, sym=packed.zeros is None, layout=packed.layout,
                has_g_idx=packed.g_idx is not None, n_groups=packed.num_groups)
        with torch.no_grad():
            m.qweight.copy_(packed.qweight)
            m.scales.copy_(packed.scales)
            if packed.zeros is not None:
                m.zeros.copy_(packed.zeros)
            if packed.g_idx is not None:
                m.g_idx.copy_(packed.g_idx)
            if bias is not None:
                m.bias.data = bias.detach().clone()
        m.prepare()
        return m

    def prepare(self) -> KernelW4A16Linear:
        """Precompute repack / act-order sort so forward is sync-free (runs after load_state_dict and ``.to()``)."""
        if self.g_idx is not None or self.layout.kind != KIND_PORTABLE:
            try:
                prepare_w4(self.packed())
            except Exception as e:  # noqa: BLE001 - never break loading; forward computes lazily outside capture
                log.debug("W4 prepare failed: %s", e)
        return self

    def _apply(self, fn, *args, **kwargs):  # noqa: ANN001
        out = super()._apply(fn, *args, **kwargs)
        out.prepare()
        return out

    @classmethod
    def from_dense(cls, linear: nn.Linear, *, group_size: int = 128, sym: bool = True,
                   layout: str | Layout | None = None, scale_dtype: torch.dtype = torch.float16,
                   **_: Any) -> KernelW4A16Linear:
        q, s, z = quantize_w4_rtn(linear.weight.detach(), group_size, sym=sym, scale_dtype=scale_dtype)
        return cls.from_packed(pack_w4(q, s, z, group_size, layout),
                               linear.bias.detach() if linear.bias is not None else None)

    @classmethod
    def from_shape(cls, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                   device: Any = None, **kw: Any):
        return cls(in_features, out_features, bias, dtype, device, **kw)

    def packed(self) -> PackedW4:
        return PackedW4(self.qweight, self.scales, self.zeros, self.layout, self.out_features, self.in_features,
                        self.group_size, self.g_idx, self._packed_meta)

    def dequantize(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        return self.packed().dequantize(dtype or torch.float32)

    def quant_spec(self) -> dict[str, Any]:
        return {"bits": 4, "group_size": self.group_size, "sym": self.sym, "layout": self.layout.id,
                "has_g_idx": self.g_idx is not None, "n_groups": int(self.scales.shape[0])}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return w4a16_linear(x, self.packed(), self._bias(x))


class KernelFp8Linear(_KernelLinear):
    """FP8 e4m3fn weights (per_channel / per_tensor / 128x128 block2d scales), dynamic FP8 activations."""

    kind: ClassVar[str] = "fp8"

    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                 device: Any = None, *, granularity: str = "per_channel", block: int = 128, **_: Any):
        super().__init__(in_features, out_features, bias, dtype, device)
        if granularity not in ("per_tensor", "per_channel", "block2d"):
            raise ConfigError(f"unknown fp8 weight granularity {granularity!r}")
        self.granularity, self.block = granularity, int(block)
        sshape = {"per_tensor": (1,), "per_channel": (out_features,),
                  "block2d": (-(-out_features // block), -(-in_features // block))}[granularity]
        self.register_buffer("weight_fp8", torch.zeros((out_features, in_features), dtype=torch.float8_e4m3fn,
                                                       device=device))
        self.register_buffer("weight_scale", torch.ones(sshape, dtype=torch.float32, device=device))

    @classmethod
    def from_dense(cls, linear: nn.Linear, *, granularity: str = "per_channel", block: int = 128,
                   **_: Any) -> KernelFp8Linear:
        m = cls(linear.in_features, linear.out_features, linear.bias is not None, linear.weight.dtype,
                linear.weight.device, granularity=granularity, block=block)
        q, s = quantize_weight_fp8(linear.weight.detach(), granularity, block)
        with torch.no_grad():
            m.weight_fp8.copy_(q)
            m.weight_scale.copy_(s.reshape(m.weight_scale.shape))
            if linear.bias is not None:
                m.bias.copy_(linear.bias.detach().to(m.bias.dtype))
        return m

    @classmethod
    def from_shape(cls, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                   device: Any = None, **kw: Any):
        return cls(in_features, out_features, bias, dtype, device, **kw)

    def quant_spec(self) -> dict[str, Any]:
        return {"granularity": self.granularity, "block": self.block}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return fp8_linear(x, self.weight_fp8, self.weight_scale, self._bias(x), block=self.block)


class KernelInt8Linear(_KernelLinear):
    """INT8 W8A8 (per-channel weight scale, dynamic per-token activation scale)."""

    kind: ClassVar[str] = "int8"

    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                 device: Any = None, **_: Any):
        super().__init__(in_features, out_features, bias, dtype, device)
        self.register_buffer("weight_int8", torch.zeros((out_features, in_features), dtype=torch.int8, device=device))
        self.register_buffer("weight_scale", torch.ones(out_features, dtype=torch.float32, device=device))

    @classmethod
    def from_dense(cls, linear: nn.Linear, **_: Any) -> KernelInt8Linear:
        m = cls(linear.in_features, linear.out_features, linear.bias is not None, linear.weight.dtype,
                linear.weight.device)
        q, s = quantize_act_int8(linear.weight.detach())  # per output channel == per row of W
        with torch.no_grad():
            m.weight_int8.copy_(q)
            m.weight_scale.copy_(s)
            if linear.bias is not None:
                m.bias.copy_(linear.bias.detach().to(m.bias.dtype))
        return m

    @classmethod
    def from_shape(cls, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                   device: Any = None, **kw: Any):
        return cls(in_features, out_features, bias, dtype, device, **kw)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return int8_linear(x, self.weight_int8, self.weight_scale, self._bias(x))


class KernelW8A16Linear(_KernelLinear):
    """8-bit weight-only linear backed by :func:`w8a16_linear` (``forge/kernels/ops_gemm.py:843-887``; buffers
    ``qweight int8 [N, K]`` and ``scales [G, N]``)."""

    kind: ClassVar[str] = "w8a16"

    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                 device: Any = None, *, group_size: int = -1, **_: Any):
        super().__init__(in_features, out_features, bias, dtype, device)
        self.group_size = int(group_size)
        g = num_groups(in_features, group_size)
        self.register_buffer("qweight", torch.zeros((out_features, in_features), dtype=torch.int8, device=device))
        self.register_buffer("scales", torch.zeros((g, out_features), dtype=dtype or torch.float16, device=device))

    @classmethod
    def from_packed(cls, packed: PackedW8, bias: torch.Tensor | None = None) -> KernelW8A16Linear:
        m = cls(packed.k, packed.n, bias is not None, packed.scales.dtype, packed.qweight.device,
                group_size=packed.group_size)
        with torch.no_grad():
            m.qweight.copy_(packed.qweight)
            m.scales.copy_(packed.scales)
            if bias is not None:
                m.bias.data = bias.detach().clone()
        return m

    @classmethod
    def from_dense(cls, linear: nn.Linear, *, group_size: int = -1, scale_dtype: torch.dtype = torch.float16,
                   **_: Any) -> KernelW8A16Linear:
        q, s = quantize_w8_rtn(linear.weight.detach(), group_size, scale_dtype)
        return cls.from_packed(pack_w8(q, s, group_size), linear.bias.detach() if linear.bias is not None else None)

    @classmethod
    def from_shape(cls, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                   device: Any = None, **kw: Any):
        return cls(in_features, out_features, bias, dtype, device, **kw)

    def packed(self) -> PackedW8:
        return PackedW8(self.qweight, self.scales, PORTABLE_W8, self.out_features, self.in_features, self.group_size)

    def dequantize(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        return self.packed().dequantize(dtype or torch.float32)

    def quant_spec(self) -> dict[str, Any]:
        return {"bits": 8, "group_size": self.group_size, "layout": PORTABLE_W8.id}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return w8a16_linear(x, self.packed(), self._bias(x))


PACKED_LINEAR_CLASSES: dict[str, type] = {"w4a16": KernelW4A16Linear, "w8a16": KernelW8A16Linear,
                                          "fp8": KernelFp8Linear, "int8": KernelInt8Linear}


def make_packed_linear(kind: str, linear: nn.Linear | None = None, *, packed: PackedW4 | PackedW8 | None = None,
                       bias: torch.Tensor | None = None, in_features: int | None = None,
                       out_features: int | None = None, **kw: Any) -> nn.Module:
    """Factory of kernel-backed packed linears (``forge/kernels/ops_gemm.py:1025-1068``, GEMM-family kinds)."""
    cls = PACKED_LINEAR_CLASSES.get(kind)
    if cls is None:
        raise ConfigError(f"unknown packed linear kind {kind!r}; choose from {sorted(PACKED_LINEAR_CLASSES)}")
    if packed is not None:
        if isinstance(packed, PackedW4) and cls is KernelW4A16Linear:
            return cls.from_packed(packed, bias)
        if isinstance(packed, PackedW8) and cls is KernelW8A16Linear:
            return cls.from_packed(packed, bias)
        raise ConfigError(f"packed data of type {type(packed).__name__} does not match kind {kind!r}")
    if linear is not None:
        return cls.from_dense(linear, **kw)
    if in_features is None or out_features is None:
        raise ConfigError("give a dense `linear`, `packed` data, or in_features/out_features")
    return cls.from_shape(in_features, out_features, bias is not None, **kw)


__all__ = [
    "KernelFp8Linear", "KernelInt8Linear", "KernelW4A16Linear", "KernelW8A16Linear", "PACKED_LINEAR_CLASSES",
    "force_ref", "forced_impl", "fp8_linear", "int8_gemm", "int8_linear", "kernel_debug", "kernel_strict",
    "last_path", "make_packed_linear", "prepare_fp8_scales", "prepare_w4", "quantize_act_fp8", "quantize_act_int8",
    "quantize_weight_fp8", "reset_failure_memo", "w4_dequant", "w4a16_linear", "w8a16_linear",
]
