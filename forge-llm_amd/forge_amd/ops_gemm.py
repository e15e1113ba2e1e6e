"""GEMM-family ops and packed-linear modules of the quantized-linear path, computed by libforge_mi355x.so only.

The public surface is the reference's ``forge/kernels/ops_gemm.py`` (``w4a16_linear`` :287-317, ``w8a16_linear``
:320-346, ``quantize_act_fp8`` :359-388, ``quantize_weight_fp8`` :391-393, ``fp8_linear`` :396-461,
``quantize_act_int8`` :467-480, ``int8_linear`` :483-515, ``prepare_w4`` :267-277, ``Kernel*Linear`` :769-961,
``make_packed_linear`` :1025-1068): same names, arguments, defaults, output dtypes, error types and module buffer
names, so callers and stored state dicts work unchanged.  Underneath, every op is one call into the C ABI
(``include/forge_mi355x.h``) on the caller's current stream.

Where this build differs on purpose:

* One path.  ``last_path(op)`` is ``"hip"``.  A tensor off the GPU, a missing library, ``FORGE_FORCE_REF=1`` or a
  failed launch raises; nothing falls back to a torch oracle (``FORGE_KERNEL_STRICT=1`` behaviour, always).
* Each device runs a known-answer self-test of the kernels the first time an op meets it (``device_selftest``):
  inputs built so that every partial sum is exact, so the expected outputs hold bit for bit whatever the kernel's
  summation order.  A failure raises ``KernelCorrectnessError``.
* Launches never synchronise and allocate only from torch's caching allocator on the current stream (outputs, the
  split-K workspace), so they can be captured in a HIP graph.
"""
from __future__ import annotations

import logging
import os
import threading
from dataclasses import dataclass
from typing import Any, Callable, ClassVar

import torch
import torch.nn as nn

from . import _lib
from .errors import ConfigError, HardwareUnsupported, KernelCorrectnessError
from .layouts import (
    CDNA4_W4,
    KIND_CDNA4,
    KIND_PORTABLE,
    MISSING_SORT,
    PORTABLE_W4,
    PORTABLE_W8,
    Layout,
    PackedW4,
    PackedW8,
    cached_group_sort,
    get_layout,
    num_groups,
    pack_w4,
    pack_w8,
    quantize_fp8_weight,
    quantize_int8_weight,
    quantize_w4_rtn,
    quantize_w8_rtn,
    repack,
    sz8_blocks,
    w4_storage_shapes,
)

log = logging.getLogger("forge_amd.ops_gemm")

FP8_E4M3_MAX = 448.0
_PATHS: dict[str, str] = {}
_ONCE: set[str] = set()
_ONCE_LOCK = threading.Lock()


# ================================================================================================ switches
def force_ref() -> bool:
    """``FORGE_FORCE_REF=1``: the caller asks for the torch oracle, which this build does not ship (ops raise)."""
    return os.environ.get("FORGE_FORCE_REF", "0") == "1"


def kernel_debug() -> bool:
    return os.environ.get("FORGE_KERNEL_DEBUG", "0") == "1"


def kernel_strict() -> bool:
    """Kernel failures always raise in this build: there is no second path to serve the call."""
    return True


def last_path(op: str) -> str | None:
    """The path the last call of ``op`` took: ``"hip"`` (or None before the first call)."""
    return _PATHS.get(op)


def last_kernel() -> str:
    """The kernel, with its launch form, that this thread's last op ran (``fg_last_kernel``): finer than
    :func:`last_path`, which names the path only."""
    return _lib.last_kernel()


def reset_failure_memo() -> None:
    """API compatibility: nothing is memoised, since no failure is ever routed around."""


def _done(op: str) -> None:
    _PATHS[op] = "hip"
    if kernel_debug():
        log.info("%s -> hip", op)


def _warn_once(key: str, message: str) -> None:
    with _ONCE_LOCK:
        fresh = key not in _ONCE
        _ONCE.add(key)
    if fresh:
        log.warning(message)


# ================================================================================================ plumbing
def _ld(t: torch.Tensor) -> int:
    """Row stride handed to the C ABI.  torch calls a one-row tensor contiguous whatever its dim-0 stride, which
    can then be smaller than the row; the row length is the safe stride there."""
    return int(t.stride(0)) if t.shape[0] > 1 else int(t.shape[1])


def _as_rows(x: torch.Tensor) -> torch.Tensor:
    """``x [..., K]`` as ``[M, K]`` with unit stride along K and rows that do not overlap (copied only if not)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) == 1 and (x2.shape[0] <= 1 or x2.stride(0) >= x2.shape[1]):
        return x2
    return x2.contiguous()


def _unit_stride(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _check(status: int, op: str) -> None:
    _lib.check(status, op)


def _code_or_zero(t: torch.Tensor | None) -> int:
    return 0 if t is None else _lib.dtype_code(t.dtype)


def _capturing(t: torch.Tensor) -> bool:
    try:
        return bool(t.is_cuda and torch.cuda.is_current_stream_capturing())
    except RuntimeError:
        return False


def _device_index(t: torch.Tensor) -> int:
    return t.device.index if t.device.index is not None else torch.cuda.current_device()


def _on_gpu(t: torch.Tensor, op: str) -> None:
    """Raise unless ``t`` is on a gfx950 GPU whose self-test passed (run here on first sight of a device)."""
    if force_ref():
        raise HardwareUnsupported(f"{op}: FORGE_FORCE_REF=1 asks for the torch reference path, which forge_amd does "
                                  "not include (run the reference implementation for that)")
    _lib.require_device(t, op)
    _SELFTEST.ensure(t)


# ================================================================================================ device self-test
class _SelfTest:
    """Known-answer checks of the W4A16, INT8 and FP8 kernels, once per device (the reference gates its native
    kernels on a one-time numerical self-test, ``forge/kernels/ops_gemm.py:626-652``).

    Inputs are small integers times powers of two, so every product and partial sum is exact in fp32 and the
    expected outputs do not depend on summation order: each kernel must reproduce them bit for bit.  No oracle is
    involved; the expected values are closed forms evaluated with integer arithmetic on the host.
    """

    def __init__(self) -> None:
        self._state: dict[int, str] = {}  # device -> "running" | "ok"
        self._lock = threading.Lock()

    def ensure(self, t: torch.Tensor) -> None:
        if os.environ.get("FORGE_AMD_SELFTEST", "1") == "0":
            return
        dev = _device_index(t)
        with self._lock:
            if self._state.get(dev) in ("running", "ok"):
                return
            if _capturing(t):  # cannot synchronise under capture; the next eager call runs it
                return
            self._state[dev] = "running"
        try:
            failures = self.run(torch.device("cuda", dev))
        except BaseException:
            with self._lock:
                self._state.pop(dev, None)
            raise
        with self._lock:
            if failures:
                self._state.pop(dev, None)
            else:
                self._state[dev] = "ok"
        if failures:
            raise KernelCorrectnessError(f"forge_amd self-test failed on cuda:{dev}: {'; '.join(failures)}",
                                         details={"device": dev, "failures": failures})

    @staticmethod
    def run(dev: torch.device) -> list[str]:
        with torch.cuda.device(dev):
            stream = torch.cuda.Stream(dev)
            stream.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(stream):
                bad = []
                for name, fn in (("w4a16", _selftest_w4), ("int8", _selftest_int8), ("fp8", _selftest_fp8)):
                    if not fn(dev):
                        bad.append(name)
            torch.cuda.current_stream(dev).wait_stream(stream)
            stream.synchronize()
        return bad


_SELFTEST = _SelfTest()


def device_selftest(device: int | torch.device | None = None) -> list[str]:
    """Run the known-answer self-test on ``device`` now; returns the names of the failed checks ([] = all good)."""
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else torch.device(device).index or 0)
    return _SelfTest.run(dev)


def _selftest_w4(dev: torch.device) -> bool:
    # codes (n + 3k) % 16, zero-points (n + g) % 16, scales 2^-(n % 4), x = (k % 7) - 3: y[m, n] exact in fp32
    n, k, gs = 96, 512, 128
    nn_ = torch.arange(n).view(-1, 1)
    kk = torch.arange(k).view(1, -1)
    q = ((nn_ + 3 * kk) % 16).to(torch.uint8)
    z = ((nn_ + torch.arange(k // gs).view(1, -1)) % 16).to(torch.uint8)
    s = torch.pow(2.0, -(nn_ % 4).float()).expand(n, k // gs).half()
    w_int = q.long() - z.long().repeat_interleave(gs, dim=1)
    ok = True
    for m in (1, 16, 80):
        x_int = ((torch.arange(m).view(-1, 1) + kk) % 7 - 3)
        exact = (x_int @ w_int.t()).double() * s[:, 0].double().view(1, -1)
        y = w4a16_linear(x_int.to(torch.bfloat16).to(dev), pack_w4(q, s, z, gs).to(dev))
        ok &= torch.equal(y.cpu(), exact.float().to(torch.bfloat16))
    return ok


def _selftest_int8(dev: torch.device) -> bool:
    m, n, k = 64, 128, 1024
    a = ((torch.arange(m).view(-1, 1) * 7 + torch.arange(k)) % 255 - 127).to(torch.int8)
    b = ((torch.arange(n).view(-1, 1) * 5 + 3 * torch.arange(k)) % 255 - 127).to(torch.int8)
    exact = a.long() @ b.long().t()
    y = int8_gemm(a.to(dev), None, b.to(dev), None, out_dtype=torch.int32)
    return torch.equal(y.cpu().long(), exact)


def _selftest_fp8(dev: torch.device) -> bool:
    # e4m3 codes of small integers (exact), power-of-two scales: y exact in fp32
    m, n, k = 32, 64, 256
    xi = ((torch.arange(m).view(-1, 1) + torch.arange(k)) % 9 - 4).float()
    wi = ((torch.arange(n).view(-1, 1) * 3 + torch.arange(k)) % 7 - 3).float()
    sx = torch.pow(2.0, -(torch.arange(m) % 3).float())
    sw = torch.pow(2.0, -(torch.arange(n) % 5).float())
    exact = (xi.double() @ wi.double().t()) * sx.double().view(-1, 1) * sw.double().view(1, -1)
    y = fp8_linear(xi.to(torch.float8_e4m3fn).to(dev), wi.to(torch.float8_e4m3fn).to(dev), sw.to(dev),
                   x_scale=sx.to(dev), out_dtype=torch.float32)
    return torch.equal(y.cpu().double(), exact)


# ================================================================================================ W4A16
_W4_IMPLS = {"gemv": "gemv", "dot": "mfma", "mfma": "mfma", "dequant_matmul": "dequant_gemm",
             "dequant_gemm": "dequant_gemm", "prefill": "prefill", "legacy": "generic", "generic": "generic",
             "auto": None, None: None}


def forced_impl() -> str | None:
    """``FORGE_W4_IMPL`` = gemv | mfma | prefill | dequant_gemm | generic (the reference's dot / dequant_matmul / legacy
    map to mfma / dequant_gemm / generic; dequant_gemm names the prefill kernels, which fuse the dequantisation into
    the MFMA tiles); anything else means the policy."""
    return _W4_IMPLS.get(os.environ.get("FORGE_W4_IMPL", "").strip().lower())


def _w4_config(config: dict[str, Any] | None) -> _lib.W4Config | None:
    """The C launch knobs of a W4A16 / W8A16 ``config`` dict (None = the built-in per-shape policy)."""
    c = dict(config or {})
    if c.get("impl") not in _W4_IMPLS:
        raise ConfigError(f"unknown W4A16 impl {c.get('impl')!r}: use gemv, mfma, prefill or generic")
    if c.get("gemv_kernel") not in _lib.GEMV_KERNEL:
        raise ConfigError(f"unknown GEMV kernel {c.get('gemv_kernel')!r}: use split, tile or wave")
    impl = forced_impl() or _W4_IMPLS[c.get("impl")]
    if impl is None and not c:
        return None
    knobs = [int(c.get(key) or 0) for key in ("rows_per_wave", "max_blocks", "tile_m", "split_k", "tile_n")]
    return _lib.W4Config(_lib.W4_IMPL[impl], *knobs, _lib.GEMV_KERNEL[c.get("gemv_kernel")])


def _cfg_ref(cfg: Any) -> Any:
    return None if cfg is None else _lib.ctypes.byref(cfg)


def _layout_copy(packed: PackedW4, lay: Layout) -> PackedW4:
    """``packed`` in ``lay``: itself, or a repacked copy kept in ``packed.meta`` until its tensors change."""
    if packed.layout.id == lay.id:
        return packed
    stamp = tuple((t.data_ptr(), t._version) for t in packed.tensors().values())
    copies = packed.meta.setdefault("hip.layout_copies", {})
    hit = copies.get(lay.id)
    if hit is None or hit[0] != stamp:
        hit = copies[lay.id] = (stamp, repack(packed, lay))
    return hit[1]


def prepare_w4(packed: PackedW4, layout: Layout | str | None = None) -> PackedW4:
    """Do the host-synchronising preparation of a W4 weight up front (``forge/kernels/ops_gemm.py:267-277``): the
    repack of an mma_fragment artifact to portable_row, the act-order column sort; with ``layout`` (e.g.
    ``CDNA4_W4``), the repack into that layout.  Call after loading or moving a weight, outside graph capture;
    returns the weight the kernels will read."""
    if layout is not None:
        lay = get_layout(layout) if isinstance(layout, str) else layout
        packed = _layout_copy(packed, lay)
        if lay.kind == KIND_CDNA4:
            return packed
    p = _layout_copy(packed, PORTABLE_W4) if packed.layout.kind != KIND_CDNA4 else packed
    if p.g_idx is not None:
        cached_group_sort(p, compute=True)
    return p


# Rows for which a portable_row weight's 8-channel scale blocks (kept by KernelW4A16Linear.prepare) serve the call:
# the split-K decode GEMV's, which reads them as one contiguous run per wavefront and K slice (graph replays over a
# 1.2 GB ring, M = 1, us, portable / blocked: qkv 5.13 / 4.89, o_proj 4.31 / 4.26, gate+up 13.84 / 12.91 (12.4 once
# the blocked form took two channel blocks per workgroup), down 9.16 / 8.59; M = 2 down 11.29 / 10.15), bit-identical
# results.
SZ8_ROWS = 2
_SZ8_KEY = "hip.sz8"  # p.meta entry: (tensor stamp, scales8, zeros8)


def _stamp(packed: PackedW4) -> tuple:
    return tuple((t.data_ptr(), t._version) for t in packed.tensors().values())


def prepare_w4_sz8(packed: PackedW4) -> bool:
    """Keep ``packed``'s scales and zero words re-blocked by 8 channels (``layouts.sz8_blocks``) in ``packed.meta``
    for the 1..2-row decode GEMV; True when made (a portable_row weight on the GPU with N % 8 == 0, K % 32 == 0, a
    group size that is a multiple of 32 or one group, 16-bit scales, no g_idx).  Outside graph capture."""
    if not _sz8_eligible(packed):
        return False
    s8, z8 = sz8_blocks(packed.scales, packed.zeros, packed.n)
    packed.meta[_SZ8_KEY] = (_stamp(packed), s8, z8)
    return True


def _sz8_eligible(p: PackedW4) -> bool:
    return (p.layout.kind == KIND_PORTABLE and p.qweight.is_cuda and p.g_idx is None and p.n % 8 == 0
            and p.k % 32 == 0 and (p.group_size <= 0 or p.group_size >= p.k or p.group_size % 32 == 0)
            and p.scales.dtype in (torch.float16, torch.bfloat16) and p.num_groups == num_groups(p.k, p.group_size))


def _sz8_copy(packed: PackedW4) -> tuple[torch.Tensor, torch.Tensor | None] | None:
    """The 8-channel scale blocks kept beside a portable_row weight, if made and its tensors have not changed."""
    hit = packed.meta.get(_SZ8_KEY) if packed.meta is not None else None
    return (hit[1], hit[2]) if hit is not None and hit[0] == _stamp(packed) else None


def _w4_sz8_call(x2: torch.Tensor, p: PackedW4, blocks: tuple[torch.Tensor, torch.Tensor | None],
                 bias: torch.Tensor | None, y: torch.Tensor) -> bool:
    """The decode GEMV on the 8-channel scale blocks; False (nothing launched) when x's alignment rules it out."""
    if _ld(x2) % 8 or x2.data_ptr() % 16 or _ld(p.qweight) % 4 or p.qweight.data_ptr() % 16:
        return False
    m, k = x2.shape
    s8, z8 = blocks
    _check(_lib.lib().fg_w4a16_gemv_sz8(
        _lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(p.qweight), _ld(p.qweight), _lib.ptr(s8),
        _lib.dtype_code(s8.dtype), _lib.ptr(z8), _lib.ptr(bias), _code_or_zero(bias), _lib.ptr(y), y.stride(0), m, p.n,
        k, p.group_size, p.num_groups, _lib.stream_of(x2)), "fg_w4a16_gemv_sz8")
    return True


@dataclass
class _W4Operands:
    weight: PackedW4
    perm: torch.Tensor | None = None
    g_idx: torch.Tensor | None = None


def _w4_operands(packed: PackedW4, capturing: bool) -> _W4Operands:
    """What the portable-row kernels read: the portable weight, plus either the sorted weight and its column
    permutation (regular act order) or the per-column ``g_idx`` (irregular act order, or a cold cache under
    capture)."""
    p = _layout_copy(packed, PORTABLE_W4)
    if p.g_idx is None:
        return _W4Operands(p)
    sorted_ = cached_group_sort(p, compute=not capturing)
    if sorted_ is MISSING_SORT:
        _warn_once("w4_capture", "act-order W4 weight met graph capture unprepared (call prepare_w4 first): the "
                                 "per-column g_idx kernel serves it")
    if not sorted_:
        return _W4Operands(p, g_idx=p.g_idx)
    return _W4Operands(sorted_[0], perm=sorted_[1])


def _w4_call(x2: torch.Tensor, ops_: _W4Operands, bias: torch.Tensor | None, y: torch.Tensor,
             cfg: _lib.W4Config | None) -> None:
    L = _lib.lib()
    w = ops_.weight
    m, k = x2.shape
    x_ok = int(_ld(x2) % 8 == 0 and x2.data_ptr() % 16 == 0)
    q_ok = int(_ld(w.qweight) % 4 == 0 and w.qweight.data_ptr() % 16 == 0)
    ws_bytes = L.fg_w4a16_workspace_bytes(m, w.n, k, w.group_size, x_ok, q_ok, int(ops_.g_idx is not None),
                                          _cfg_ref(cfg))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x2.device) if ws_bytes else None
    z = w.zeros
    _check(L.fg_w4a16_gemm(
        _lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(w.qweight), _ld(w.qweight), _lib.ptr(w.scales),
        _lib.dtype_code(w.scales.dtype), _ld(w.scales), _lib.ptr(z), 0 if z is None else _ld(z), _lib.ptr(ops_.perm),
        _lib.ptr(ops_.g_idx), _lib.ptr(bias), _code_or_zero(bias), _lib.ptr(y), y.stride(0), m, w.n, k, w.group_size,
        w.num_groups, _cfg_ref(cfg), _lib.ptr(ws), ws_bytes, _lib.stream_of(x2)), "fg_w4a16_gemm")


def _cdna4_fits(p: PackedW4, m: int, config: dict[str, Any] | None) -> bool:
    """Whether the CDNA4-layout kernel serves this call (else the weight's portable copy does)."""
    impl = forced_impl() or _W4_IMPLS.get((config or {}).get("impl"))
    return (p.layout.kind == KIND_CDNA4 and 1 <= m <= 64 and p.g_idx is None and p.k % 128 == 0
            and (p.group_size <= 0 or p.group_size % 128 == 0) and p.scales.dtype in (torch.float16, torch.bfloat16)
            and impl in (None, "mfma"))


# Rows for which a portable_row weight's CDNA4-layout copy (kept by KernelW4A16Linear.prepare) serves the call: its MFMA
# kernels beat the portable_row policy there (graph replays, us, portable / CDNA4: M = 16 qkv 10.2 / 8.8, o_proj 8.2 /
# 7.5, gate+up 22.1 / 18.0, down 15.8 / 14.4; M = 64 17.6 / 16.7, 14.4 / 13.8, 35.9 / 32.5, 25.2 / 23.6); one or two
# rows stay on the split-K GEMV.
CDNA4_COPY_ROWS = (3, 64)


def _cdna4_copy(packed: PackedW4) -> PackedW4 | None:
    """The CDNA4-layout copy kept beside a portable_row weight, if one was made and its tensors have not changed."""
    copies = packed.meta.get("hip.layout_copies") if packed.meta is not None else None
    hit = copies.get(CDNA4_W4.id) if copies else None
    if hit is None:
        return None
    return hit[1] if hit[0] == tuple((t.data_ptr(), t._version) for t in packed.tensors().values()) else None


def _w4_cdna4_call(x2: torch.Tensor, p: PackedW4, bias: torch.Tensor | None, y: torch.Tensor) -> None:
    m, k = x2.shape
    z = p.zeros
    L = _lib.lib()
    ws_bytes = L.fg_w4a16_cdna4_workspace_bytes(m, p.n, k, p.group_size)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x2.device) if ws_bytes else None
    _check(L.fg_w4a16_gemm_cdna4(
        _lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(p.qweight), _ld(p.qweight), _lib.ptr(p.scales),
        _lib.dtype_code(p.scales.dtype), _ld(p.scales), _lib.ptr(z), 0 if z is None else _ld(z), _lib.ptr(bias),
        _code_or_zero(bias), _lib.ptr(y), y.stride(0), m, p.n, k, p.group_size, p.num_groups, _lib.ptr(ws), ws_bytes,
        _lib.stream_of(x2)), "fg_w4a16_gemm_cdna4")


def w4a16_linear(x: torch.Tensor, packed: PackedW4, bias: torch.Tensor | None = None, *,
                 config: dict[str, Any] | None = None, deterministic: bool = True) -> torch.Tensor:
    """``y = x @ dequant(W)^T (+ bias)`` for bf16 / fp16 ``x [..., K]`` on a gfx950 GPU; returns ``x.dtype``.

    The C library picks the kernel per shape (``config={"impl": "gemv" | "mfma" | "prefill" | "generic", ...}`` or
    ``FORGE_W4_IMPL`` overrides it): split-K register GEMV for 1-2 rows (and small weights at 3-4), the skinny MFMA
    kernel up to 32 rows, dequantise-to-LDS MFMA tiles beyond, a per-element kernel for irregular act order or
    unaligned weights.  A weight in the ``cdna4_mfma`` layout (``prepare_w4(p, CDNA4_W4)``) runs its own MFMA kernels
    for 1..64 rows (a register ring, or an LDS ring with a K-split reduce for 33..64 rows and long K) and a
    portable_row copy beyond.  Every kernel reduces in a fixed order, so results are run-to-run reproducible whatever
    ``deterministic`` says.
    """
    _on_gpu(x, "w4a16_linear")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise HardwareUnsupported(f"w4a16_linear: activations must be bf16 or fp16, got {x.dtype}")
    if x.shape[-1] != packed.k:
        raise ConfigError(f"x has K={x.shape[-1]}, the packed weight K={packed.k}")
    if packed.qweight.device != x.device:
        raise ConfigError(f"the weight is on {packed.qweight.device}, x on {x.device}")
    x2 = _as_rows(x)
    m = x2.shape[0]
    y = torch.empty((m, packed.n), dtype=x.dtype, device=x.device)
    if m:
        b = None if bias is None else bias.contiguous()
        copy = (_cdna4_copy(packed) if packed.layout.kind == KIND_PORTABLE
                and CDNA4_COPY_ROWS[0] <= m <= CDNA4_COPY_ROWS[1] else None)
        blocks = (_sz8_copy(packed) if packed.layout.kind == KIND_PORTABLE and m <= SZ8_ROWS and config is None
                  and forced_impl() is None else None)
        if blocks is not None and _w4_sz8_call(x2, packed, blocks, b, y):
            pass
        elif copy is not None and _cdna4_fits(copy, m, config):
            _w4_cdna4_call(x2, copy, b, y)
        elif _cdna4_fits(packed, m, config):
            _w4_cdna4_call(x2, packed, b, y)
        else:
            if packed.layout.kind == KIND_CDNA4:
                _warn_once("cdna4_copy", "a cdna4_mfma W4 weight met a call its kernel does not take (more than 64 rows, "
                                         "a forced impl, or its shape): a portable_row copy serves it and is kept")
            _w4_call(x2, _w4_operands(packed, _capturing(x2)), b, y, _w4_config(config))
    _done("w4a16_linear")
    return y.reshape(*x.shape[:-1], packed.n)


def w4_dequant(packed: PackedW4, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Dense ``[N, K]`` weight on the GPU (``fg_w4_dequant``): ``(q - z) * s`` in fp32, rounded once to ``dtype``."""
    p = _layout_copy(packed, PORTABLE_W4)
    _on_gpu(p.qweight, "w4_dequant")
    if dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ConfigError(f"w4_dequant: no {dtype} output")
    out = torch.empty((p.n, p.k), dtype=dtype, device=p.qweight.device)
    z = p.zeros
    _check(_lib.lib().fg_w4_dequant(
        _lib.ptr(p.qweight), _ld(p.qweight), _lib.ptr(p.scales), _lib.dtype_code(p.scales.dtype), _ld(p.scales),
        _lib.ptr(z), 0 if z is None else _ld(z), _lib.ptr(p.g_idx), _lib.ptr(out), _lib.dtype_code(dtype),
        out.stride(0), p.n, p.k, p.group_size, p.num_groups, _lib.stream_of(out)), "fg_w4_dequant")
    _done("w4_dequant")
    return out


# ================================================================================================ W8A16
def w8a16_linear(x: torch.Tensor, packed: PackedW8, bias: torch.Tensor | None = None, *,
                 config: dict[str, Any] | None = None, deterministic: bool = True) -> torch.Tensor:
    """``y = x @ (q * s)^T (+ bias)`` with symmetric int8 weights (``forge/kernels/ops_gemm.py:320-346``) for bf16 /
    fp16 ``x [..., K]``; returns ``x.dtype``.  A split-K GEMV for 1..4 rows, the LDS-ring and skinny MFMA kernels up
    to 64 rows, the dequantise-into-MFMA prefill kernels beyond (the ping-pong kernel on large problems), a generic
    kernel for shapes none of them takes (``config={"impl": "gemv" | "mfma" | "prefill" | "dequant_gemm" |
    "generic"}`` overrides; "dequant_gemm" names the prefill kernels); fixed-order reductions throughout."""
    _on_gpu(x, "w8a16_linear")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise HardwareUnsupported(f"w8a16_linear: activations must be bf16 or fp16, got {x.dtype}")
    if packed.layout.bits != 8:
        raise ConfigError(f"layout {packed.layout_id} is not an 8-bit layout")
    if x.shape[-1] != packed.k:
        raise ConfigError(f"x has K={x.shape[-1]}, the packed weight K={packed.k}")
    if packed.qweight.device != x.device:
        raise ConfigError(f"the weight is on {packed.qweight.device}, x on {x.device}")
    x2 = _as_rows(x)
    m = x2.shape[0]
    y = torch.empty((m, packed.n), dtype=x.dtype, device=x.device)
    if m:
        q, sc = _unit_stride(packed.qweight), _unit_stride(packed.scales)
        b = None if bias is None else bias.contiguous()
        cfg = _w4_config(config)
        L = _lib.lib()
        ws_bytes = L.fg_w8a16_workspace_bytes(m, packed.n, packed.k, packed.group_size, _cfg_ref(cfg))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
        _check(L.fg_w8a16_gemm(
            _lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(q), _ld(q), _lib.ptr(sc),
            _lib.dtype_code(sc.dtype), _ld(sc), _lib.ptr(b), _code_or_zero(b), _lib.ptr(y), y.stride(0), m, packed.n,
            packed.k, packed.group_size, packed.num_groups, _cfg_ref(cfg), _lib.ptr(ws), ws_bytes,
            _lib.stream_of(x2)), "fg_w8a16_gemm")
    _done("w8a16_linear")
    return y.reshape(*x.shape[:-1], packed.n)


# ================================================================================================ FP8
def _scale_vector(s: torch.Tensor, rows: int | None = None) -> torch.Tensor:
    """A ``[rows, 1]`` / ``[1, rows]`` (or, without ``rows``, any ``[R, 1]``) scale as a flat fp32 vector; other
    shapes unchanged (in fp32)."""
    s = s.float()
    if s.dim() == 2 and s.numel() > 1:
        if (rows is None and s.shape[1] == 1) or (rows is not None and rows in s.shape and 1 in s.shape):
            return s.reshape(-1)
    return s


@dataclass
class _ScaleSide:
    """One operand's scale as the kernel reads it: ``t[i * si + kb * sk]`` (strides in elements, 0 broadcasts);
    ``div`` groups ``div`` rows per scale row (128 x 128 weight blocks)."""

    t: torch.Tensor
    si: int
    sk: int
    div: int = 1
    blocked: bool = False
    scalar: bool = False


def _act_side(sx: torch.Tensor, m: int, kb: int) -> _ScaleSide:
    if sx.dim() == 2:
        if sx.shape[0] != m or sx.shape[1] < kb:
            raise ValueError(f"a 2-D activation scale must be [M={m}, >= {kb}], got {tuple(sx.shape)}")
        return _ScaleSide(sx, sx.stride(0), sx.stride(1), blocked=True)
    if sx.numel() == 1:
        return _ScaleSide(sx.reshape(1), 0, 0, scalar=True)
    if sx.numel() == m:
        return _ScaleSide(sx.reshape(-1), 1, 0)
    raise ValueError(f"the activation scale has {sx.numel()} entries for M={m}")


def _weight_side(sw: torch.Tensor, n: int, kb: int, block: int) -> _ScaleSide:
    if sw.dim() == 2:
        if sw.shape[1] < kb:
            raise ValueError(f"a 2-D weight scale needs >= {kb} columns, got {tuple(sw.shape)}")
        if sw.shape[0] == n:
            return _ScaleSide(sw, sw.stride(0), sw.stride(1), 1, blocked=True)
        if sw.shape[0] >= -(-n // block):
            return _ScaleSide(sw, sw.stride(0), sw.stride(1), block, blocked=True)
        raise ValueError(f"a 2-D weight scale has {sw.shape[0]} rows for N={n} with block {block}")
    if sw.numel() == 1:
        return _ScaleSide(sw.reshape(1), 0, 0, scalar=True)
    if sw.numel() == n:
        return _ScaleSide(sw.reshape(-1), 1, 0)
    raise ValueError(f"the weight scale has {sw.numel()} entries for N={n}")


def prepare_fp8_scales(sx: torch.Tensor, sw: torch.Tensor, m: int, n: int, k: int, block: int):
    """The kernel's view of any accepted scale combination (the rules of ``forge/kernels/triton/gemm_fp8.py:151-191``):
    ``(mode, sa, sb, (sa_m, sa_k, sb_n, sb_k), sb_div)`` with element strides (0 broadcasts).  Mode 0: both scales
    per tensor; 1: per token and / or per channel; 2: either side K-blocked (1 x ``block`` activations,
    ``block`` x ``block`` or per-channel-per-block weights).  Sizes that do not fit raise ValueError."""
    kb = -(-k // block)
    a = _act_side(sx.float().contiguous(), m, kb)
    b = _weight_side(sw.float().contiguous(), n, kb, block)
    if a.scalar and b.scalar:
        return 0, a.t, b.t, (0, 0, 0, 0), block
    if not (a.blocked or b.blocked):
        return 1, a.t, b.t, (a.si, 0, b.si, 0), block
    return 2, a.t, b.t, (a.si, a.sk, b.si, b.sk), b.div


def _fp8_block_quant(x2: torch.Tensor, bm: int, bk: int, static: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor]:
    """Codes and ``[ceil(M/bm), ceil(K/bk)]`` scales (or the static scale) of a block-granular FP8 quantisation."""
    m, k = x2.shape
    q = torch.empty((m, k), dtype=torch.float8_e4m3fn, device=x2.device)
    kb = -(-k // bk)
    if static is not None:
        s_out, s = None, static.float().reshape(1).to(x2.device).contiguous()
    else:
        s_out = s = torch.empty((-(-m // bm) if m else 0, kb), dtype=torch.float32, device=x2.device)
    if m:
        _check(_lib.lib().fg_quant_fp8_block(
            _lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(q), _ld(q), _lib.ptr(s_out), kb, m, k, bm, bk,
            _lib.ptr(None if static is None else s), _lib.stream_of(x2)), "fg_quant_fp8_block")
    return q, s


def _fp8_row_quant(x2: torch.Tensor, static: torch.Tensor | None, rms_weight: torch.Tensor | None,
                   rms_eps: float | None) -> tuple[torch.Tensor, torch.Tensor]:
    m, k = x2.shape
    q = torch.empty((m, k), dtype=torch.float8_e4m3fn, device=x2.device)
    if static is not None:
        s = static.float().reshape(-1).to(x2.device)
        if s.numel() == 1:
            s = s.expand(m)
        if s.numel() != m:
            raise ConfigError(f"a static per-token scale needs M={m} entries, got {s.numel()}")
        s = s.contiguous()
        s_out, s_static = None, s
    else:
        s = s_out = torch.empty(m, dtype=torch.float32, device=x2.device)
        s_static = None
    w = None if rms_weight is None else rms_weight.contiguous()
    if m:
        _check(_lib.lib().fg_quant_fp8_rowwise(
            _lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(q), _ld(q), _lib.ptr(s_out), m, k,
            _lib.ptr(s_static), _lib.ptr(w), _code_or_zero(w), float(rms_eps or 0.0), int(rms_eps is not None),
            _lib.stream_of(x2)), "fg_quant_fp8_rowwise")
    return q, s


def quantize_act_fp8(x: torch.Tensor, *, granularity: str = "per_token", block: int = 128,
                     scale: torch.Tensor | None = None, rms_weight: torch.Tensor | None = None,
                     rms_eps: float | None = None, fmt: str = "e4m3") -> tuple[torch.Tensor, torch.Tensor]:
    """Dynamic (or static ``scale=``) OCP e4m3fn quantisation of ``x [..., K]`` -> ``(codes, fp32 scale)``.

    Scale shapes: per_token ``[M]``, per_tensor ``[1]``, block ``[M, ceil(K/block)]``, block2d
    ``[ceil(M/block), ceil(K/block)]``.  ``rms_eps`` fuses ``x * rsqrt(mean(x^2) + eps) * rms_weight`` in front of
    the per-token quantisation.  A static per-tensor scale is applied row by row (one workgroup per row); a dynamic
    per-tensor amax is reduced by many workgroups.
    """
    _on_gpu(x, "quantize_act_fp8")
    if fmt != "e4m3":
        raise HardwareUnsupported("quantize_act_fp8: gfx950 kernels here produce OCP e4m3fn only")
    if not x.is_floating_point():
        raise ConfigError("quantize_act_fp8: x must be a float tensor")
    x2 = _as_rows(x)
    m, k = x2.shape
    gran = "per_token" if granularity == "per_channel" else granularity
    if rms_eps is not None and gran != "per_token":
        raise ConfigError("the fused RMSNorm quantiser is per token only")
    if gran == "per_token":
        q, s = _fp8_row_quant(x2, scale, rms_weight, rms_eps)
    elif gran == "per_tensor" and scale is not None:
        if scale.numel() != 1:
            raise ConfigError(f"a per-tensor scale has one entry, got {scale.numel()}")
        q, _ = _fp8_row_quant(x2, scale, None, None)
        s = scale.float().reshape(1).to(x.device)
    elif gran == "per_tensor":
        q, s = _fp8_block_quant(x2, max(m, 1), k, None)
        s = s.reshape(1) if m else torch.ones(1, dtype=torch.float32, device=x.device)
    elif gran in ("block", "block2d"):
        if scale is not None and scale.numel() != 1:
            raise ConfigError("a static scale for block granularities is one value for every block")
        q, s = _fp8_block_quant(x2, 1 if gran == "block" else block, block, scale)
    else:
        raise ConfigError(f"unknown granularity {granularity!r}")
    _done("quantize_act_fp8")
    return q.reshape(x.shape), s


def quantize_weight_fp8(w: torch.Tensor, granularity: str = "per_channel",
                        block: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """Offline FP8 weight quantisation: per_tensor | per_channel | block2d -> ``(w_fp8 [N, K], scale)``.  A weight on
    the GPU goes through the device quantiser; one on the host (a checkpoint quantised before ``.to("cuda")``) through
    ``layouts.quantize_fp8_weight``, which gives the same codes and scales bit for bit."""
    if not w.is_cuda:
        if granularity not in _FP8_SCALE_SHAPES:
            raise ConfigError(f"unknown fp8 weight granularity {granularity!r}: use {sorted(_FP8_SCALE_SHAPES)}")
        return quantize_fp8_weight(w.reshape(-1, w.shape[-1]), granularity, block)
    return quantize_act_fp8(w, granularity=granularity, block=block)


def quantize_weight_int8(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel symmetric int8 weight quantisation -> ``(w_int8 [N, K], scale fp32 [N])``: the device
    per-token quantiser for a weight on the GPU (one row per channel), ``layouts.quantize_int8_weight`` on the host;
    both give the same codes and scales bit for bit."""
    if not w.is_cuda:
        return quantize_int8_weight(w.reshape(-1, w.shape[-1]))
    return quantize_act_int8(w)


def _mm_config(config: dict[str, Any] | None) -> _lib.MMConfig | None:
    if not config:
        return None
    return _lib.MMConfig(int(config.get("tile_m") or 0), int(config.get("tile_n") or 0))


def _out_dtype(requested: torch.dtype | None, x: torch.Tensor, prequantised: bool) -> torch.dtype:
    dt = requested or (torch.bfloat16 if prequantised else x.dtype)
    return dt if dt in (torch.float16, torch.bfloat16, torch.float32) else torch.bfloat16


def fp8_linear(x: torch.Tensor, w_fp8: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None = None, *,
               x_scale: torch.Tensor | None = None, act_granularity: str | None = None, block: int = 128,
               out_dtype: torch.dtype | None = None, config: dict[str, Any] | None = None) -> torch.Tensor:
    """``y = dq(quant(x)) @ dq(w)^T (+ bias)`` on gfx950's fp8 matrix cores (OCP e4m3fn, fp32 accumulation).

    ``x`` is float (quantised here: per token, per tensor when both given scales are scalars, 1 x ``block`` when
    ``w_scale`` is 2-D) or e4m3fn with ``x_scale``.  Output: ``out_dtype``, else ``x.dtype`` (bf16 for pre-quantised
    input).
    """
    sw = _scale_vector(w_scale, w_fp8.shape[0])
    preq = x.dtype in (torch.float8_e4m3fn, torch.float8_e5m2)
    odt = _out_dtype(out_dtype, x, preq)
    if preq:
        if x_scale is None:
            raise ConfigError("fp8 activations given already quantised need x_scale")
        xq, sx = x, _scale_vector(x_scale)
    else:
        if act_granularity:
            gran = act_granularity
        elif sw.dim() == 2:
            gran = "block"
        elif sw.numel() == 1 and x_scale is not None and x_scale.numel() == 1:
            gran = "per_tensor"
        else:
            gran = "per_token"
        xq, sx = quantize_act_fp8(x, granularity=gran, block=block, scale=x_scale)
    _on_gpu(xq, "fp8_linear")
    if xq.dtype != torch.float8_e4m3fn or w_fp8.dtype != torch.float8_e4m3fn:
        raise HardwareUnsupported("fp8_linear: the gfx950 kernels take float8_e4m3fn operands (no e5m2)")
    a = _as_rows(xq)
    m, k = a.shape
    n = w_fp8.shape[0]
    if w_fp8.shape[1] != k:
        raise ConfigError(f"x has K={k}, the weight K={w_fp8.shape[1]}")
    y = torch.empty((m, n), dtype=odt, device=xq.device)
    if m:
        try:
            mode, sa, sb, (sam, sak, sbn, sbk), sb_div = prepare_fp8_scales(sx.to(a.device), sw.to(a.device), m, n, k,
                                                                            block)
        except ValueError as e:
            raise ConfigError(str(e)) from e
        wq = _unit_stride(w_fp8)
        b = None if bias is None else bias.contiguous()
        _check(_lib.lib().fg_fp8_gemm(
            _lib.ptr(a), _ld(a), _lib.ptr(sa), sam, sak, _lib.ptr(wq), _ld(wq), _lib.ptr(sb), sbn, sbk, sb_div, mode,
            block, _lib.ptr(b), _code_or_zero(b), _lib.ptr(y), y.stride(0), _lib.dtype_code(odt), m, n, k,
            _cfg_ref(_mm_config(config)), _lib.stream_of(a)), "fg_fp8_gemm")
    _done("fp8_linear")
    return y.reshape(*xq.shape[:-1], n)


# ================================================================================================ INT8
def quantize_act_int8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token symmetric int8 -> ``(codes int8, scale fp32 [M])``: IEEE ``amax / 127``, round half to even."""
    _on_gpu(x, "quantize_act_int8")
    if not x.is_floating_point():
        raise ConfigError("quantize_act_int8: x must be a float tensor")
    x2 = _as_rows(x)
    m, k = x2.shape
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty(m, dtype=torch.float32, device=x.device)
    if m:
        _check(_lib.lib().fg_quant_int8_rowwise(_lib.ptr(x2), _ld(x2), _lib.dtype_code(x2.dtype), _lib.ptr(q), _ld(q),
                                                _lib.ptr(s), m, k, _lib.stream_of(x2)), "fg_quant_int8_rowwise")
    _done("quantize_act_int8")
    return q.reshape(x.shape), s


def int8_gemm(xq: torch.Tensor, sx: torch.Tensor | None, wq: torch.Tensor, sw: torch.Tensor | None,
              bias: torch.Tensor | None = None, *, out_dtype: torch.dtype = torch.bfloat16,
              config: dict[str, Any] | None = None) -> torch.Tensor:
    """The INT8 GEMM on quantised operands (the launcher ``int8_gemm_triton``, gemm_int8.py:95-137):
    ``(float(acc) * sx[m]) * sw[n] (+ bias)`` with an exact int32 ``acc``; ``out_dtype=torch.int32`` returns ``acc``
    itself (no scales, no bias)."""
    _on_gpu(xq, "int8_gemm")
    a = _as_rows(xq)
    w = wq.contiguous()
    m, k = a.shape
    n = w.shape[0]
    if w.shape[1] != k:
        raise ConfigError(f"x has K={k}, the weight K={w.shape[1]}")
    y = torch.empty((m, n), dtype=out_dtype, device=xq.device)
    if m:
        raw = out_dtype == torch.int32
        if raw and bias is not None:
            raise ConfigError("int8_gemm: no bias on the raw int32 accumulator (out_dtype=torch.int32)")
        sa = None if raw else sx.float().reshape(-1).contiguous()
        sb = None if raw else sw.float().reshape(-1).contiguous()
        if not raw and (sa.numel() not in (1, m) or sb.numel() not in (1, n)):
            raise ConfigError(f"scales of {sa.numel()} / {sb.numel()} entries for M={m} / N={n}")
        b = None if bias is None else bias.contiguous()
        _check(_lib.lib().fg_int8_gemm(
            _lib.ptr(a), _ld(a), _lib.ptr(sa), 0 if raw else sa.numel(), _lib.ptr(w), _ld(w), _lib.ptr(sb),
            0 if raw else sb.numel(), _lib.ptr(b), _code_or_zero(b), _lib.ptr(y), y.stride(0),
            _lib.dtype_code(out_dtype), m, n, k, _cfg_ref(_mm_config(config)), _lib.stream_of(a)), "fg_int8_gemm")
    return y.reshape(*xq.shape[:-1], n)


def int8_linear(x: torch.Tensor, w_int8: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None = None, *,
                x_scale: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                config: dict[str, Any] | None = None) -> torch.Tensor:
    """SmoothQuant-style W8A8 on gfx950's int8 matrix cores: float ``x`` is quantised per token here (int8 ``x``
    comes with ``x_scale``); exact int32 accumulation, fp32 epilogue ``(acc * sx) * sw (+ bias)``."""
    preq = x.dtype == torch.int8
    if preq and x_scale is None:
        raise ConfigError("int8 activations need x_scale")
    xq, sx = (x, x_scale.float()) if preq else quantize_act_int8(x)
    y = int8_gemm(xq, sx, w_int8, _scale_vector(w_scale, w_int8.shape[0]), bias,
                  out_dtype=_out_dtype(out_dtype, x, preq), config=config)
    _done("int8_linear")
    return y


# ================================================================================================ modules
_Buffers = dict[str, "tuple[tuple[int, ...], torch.dtype, float] | None"]


class _PackedLinear(nn.Module):
    """A linear layer whose weight lives in packed buffers and whose forward is one kernel-backed op.

    Subclasses declare their buffers (:meth:`_buffer_specs`: name -> ``(shape, dtype, fill)`` or None for an absent
    optional buffer), how to build from a dense ``nn.Linear`` and the op their forward runs."""

    kind: ClassVar[str] = ""

    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                 device: Any = None, **_: Any) -> None:
        super().__init__()
        self.in_features, self.out_features = int(in_features), int(out_features)
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=dtype or torch.float32, device=device))
        else:
            self.register_parameter("bias", None)
        for name, spec in self._buffer_specs(dtype).items():
            buf = None if spec is None else torch.full(spec[0], spec[2], dtype=spec[1], device=device)
            self.register_buffer(name, buf)

    def _buffer_specs(self, dtype: torch.dtype | None) -> _Buffers:
        raise NotImplementedError

    def _linear(self, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        raise NotImplementedError

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._linear(x, None if self.bias is None else self.bias.to(x.dtype))

    @classmethod
    def from_shape(cls, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                   device: Any = None, **kw: Any) -> _PackedLinear:
        return cls(in_features, out_features, bias, dtype, device, **kw)

    def _fill(self, tensors: dict[str, torch.Tensor], bias: torch.Tensor | None) -> None:
        with torch.no_grad():
            for name, t in tensors.items():
                getattr(self, name).copy_(t.reshape(getattr(self, name).shape))
            if bias is not None:
                self.bias = nn.Parameter(bias.detach().clone())

    def quant_spec(self) -> dict[str, Any]:
        return {}

    def extra_repr(self) -> str:
        return (f"kind={self.kind}, in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}")


def _after_load(module: Any, _keys: Any) -> None:
    module.prepare()


class KernelW4A16Linear(_PackedLinear):
    """4-bit weight-only linear over :func:`w4a16_linear` (buffers ``qweight / scales / zeros / g_idx`` in the
    weight's layout: portable_row, mma_fragment or cdna4_mfma)."""

    kind: ClassVar[str] = "w4a16"

    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                 device: Any = None, *, group_size: int = 128, sym: bool = True, layout: str | Layout | None = None,
                 has_g_idx: bool = False, n_groups: int | None = None, **_: Any) -> None:
        self.group_size, self.sym, self.has_g_idx = int(group_size), bool(sym), bool(has_g_idx)
        self.layout = PORTABLE_W4 if layout is None else (get_layout(layout) if isinstance(layout, str) else layout)
        self.n_groups = int(n_groups) if n_groups is not None else num_groups(in_features, group_size)
        super().__init__(in_features, out_features, bias, dtype, device)
        self._meta: dict[str, Any] = {}
        self.register_load_state_dict_post_hook(_after_load)

    def _buffer_specs(self, dtype: torch.dtype | None) -> _Buffers:
        shapes = w4_storage_shapes(self.layout, self.out_features, self.in_features, self.n_groups, not self.sym)
        return {"qweight": (shapes["qweight"], torch.int32, 0),
                "scales": (shapes["scales"], dtype or torch.float16, 0),
                "zeros": None if self.sym else (shapes["zeros"], torch.int32, 0),
                "g_idx": ((self.in_features,), torch.int32, 0) if self.has_g_idx else None}

    @classmethod
    def from_packed(cls, packed: PackedW4, bias: torch.Tensor | None = None) -> KernelW4A16Linear:
        mod = cls(packed.k, packed.n, bias is not None, packed.scales.dtype, packed.qweight.device,
                  group_size=packed.group_size, sym=packed.zeros is None, layout=packed.layout,
                  has_g_idx=packed.g_idx is not None, n_groups=packed.num_groups)
        mod._fill(packed.tensors(), bias)
        return mod.prepare()

    @classmethod
    def from_dense(cls, linear: nn.Linear, *, group_size: int = 128, sym: bool = True,
                   layout: str | Layout | None = None, scale_dtype: torch.dtype = torch.float16,
                   **_: Any) -> KernelW4A16Linear:
        q, s, z = quantize_w4_rtn(linear.weight.detach(), group_size, sym=sym, scale_dtype=scale_dtype)
        b = None if linear.bias is None else linear.bias.detach()
        return cls.from_packed(pack_w4(q, s, z, group_size, layout), b)

    def packed(self) -> PackedW4:
        return PackedW4(self.qweight, self.scales, self.zeros, self.layout, self.out_features, self.in_features,
                        self.group_size, self.g_idx, self._meta)

    def prepare(self) -> KernelW4A16Linear:
        """Host-synchronising preparation (repack, act-order sort) done now, so forward never syncs; runs after
        ``load_state_dict`` and ``.to()``.  On the GPU a portable_row weight also gets a CDNA4-layout copy for 3..64-row
        calls (``CDNA4_COPY_ROWS``) and its scales / zero words blocked by 8 channels for 1..2-row calls
        (``SZ8_ROWS``); the state dict stays portable_row (``FORGE_W4_CDNA4_COPY=0`` / ``FORGE_W4_SZ8_COPY=0`` turn
        the copies off)."""
        if self.g_idx is not None or self.layout.kind != KIND_PORTABLE:
            try:
                prepare_w4(self.packed())
            except (ConfigError, RuntimeError) as e:  # forward prepares lazily outside capture
                log.debug("W4 prepare deferred: %s", e)
        else:
            if self._cdna4_copy_wanted():
                try:
                    prepare_w4(self.packed(), CDNA4_W4)
                except (ConfigError, RuntimeError) as e:
                    log.debug("W4 CDNA4 copy not made: %s", e)
            if os.environ.get("FORGE_W4_SZ8_COPY", "1") != "0":
                prepare_w4_sz8(self.packed())
        return self

    def _cdna4_copy_wanted(self) -> bool:
        """A portable_row weight on the GPU in a shape the CDNA4-layout kernels take."""
        return (os.environ.get("FORGE_W4_CDNA4_COPY", "1") != "0" and self.qweight.is_cuda and self.g_idx is None
                and self.in_features % 128 == 0 and (self.group_size <= 0 or self.group_size % 128 == 0)
                and self.scales.dtype in (torch.float16, torch.bfloat16))

    def _apply(self, fn: Callable, *args: Any, **kwargs: Any) -> KernelW4A16Linear:
        out = super()._apply(fn, *args, **kwargs)
        out._meta = {}
        return out.prepare()

    def dequantize(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        return self.packed().dequantize(dtype or torch.float32)

    def quant_spec(self) -> dict[str, Any]:
        return {"bits": 4, "group_size": self.group_size, "sym": self.sym, "layout": self.layout.id,
                "has_g_idx": self.g_idx is not None, "n_groups": int(self.scales.shape[0])}

    def _linear(self, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        return w4a16_linear(x, self.packed(), bias)


class KernelW8A16Linear(_PackedLinear):
    """8-bit weight-only linear over :func:`w8a16_linear` (``forge/kernels/ops_gemm.py:843-887``; buffers
    ``qweight int8 [N, K]`` and ``scales [G, N]``)."""

    kind: ClassVar[str] = "w8a16"

    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                 device: Any = None, *, group_size: int = -1, **_: Any) -> None:
        self.group_size = int(group_size)
        super().__init__(in_features, out_features, bias, dtype, device)

    def _buffer_specs(self, dtype: torch.dtype | None) -> _Buffers:
        g = num_groups(self.in_features, self.group_size)
        return {"qweight": ((self.out_features, self.in_features), torch.int8, 0),
                "scales": ((g, self.out_features), dtype or torch.float16, 0)}

    @classmethod
    def from_packed(cls, packed: PackedW8, bias: torch.Tensor | None = None) -> KernelW8A16Linear:
        mod = cls(packed.k, packed.n, bias is not None, packed.scales.dtype, packed.qweight.device,
                  group_size=packed.group_size)
        mod._fill(packed.tensors(), bias)
        return mod

    @classmethod
    def from_dense(cls, linear: nn.Linear, *, group_size: int = -1, scale_dtype: torch.dtype = torch.float16,
                   **_: Any) -> KernelW8A16Linear:
        q, s = quantize_w8_rtn(linear.weight.detach(), group_size, scale_dtype)
        b = None if linear.bias is None else linear.bias.detach()
        return cls.from_packed(pack_w8(q, s, group_size), b)

    def packed(self) -> PackedW8:
        return PackedW8(self.qweight, self.scales, PORTABLE_W8, self.out_features, self.in_features, self.group_size)

    def dequantize(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        return self.packed().dequantize(dtype or torch.float32)

    def quant_spec(self) -> dict[str, Any]:
        return {"bits": 8, "group_size": self.group_size, "layout": PORTABLE_W8.id}

    def _linear(self, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        return w8a16_linear(x, self.packed(), bias)


_FP8_SCALE_SHAPES: dict[str, Callable[[int, int, int], tuple[int, ...]]] = {
    "per_tensor": lambda n, k, b: (1,),
    "per_channel": lambda n, k, b: (n,),
    "block2d": lambda n, k, b: (-(-n // b), -(-k // b)),
}


class KernelFp8Linear(_PackedLinear):
    """FP8 e4m3fn weights with per-tensor / per-channel / 128 x 128 block scales; activations quantised to FP8 on
    the fly (buffers ``weight_fp8`` and ``weight_scale``)."""

    kind: ClassVar[str] = "fp8"

    def __init__(self, in_features: int, out_features: int, bias: bool = False, dtype: torch.dtype | None = None,
                 device: Any = None, *, granularity: str = "per_channel", block: int = 128, **_: Any) -> None:
        if granularity not in _FP8_SCALE_SHAPES:
            raise ConfigError(f"unknown fp8 weight granularity {granularity!r}: use {sorted(_FP8_SCALE_SHAPES)}")
        self.granularity, self.block = granularity, int(block)
        super().__init__(in_features, out_features, bias, dtype, device)

    def _buffer_specs(self, dtype: torch.dtype | None) -> _Buffers:
        shape = _FP8_SCALE_SHAPES[self.granularity](self.out_features, self.in_features, self.block)
        return {"weight_fp8": ((self.out_features, self.in_features), torch.float8_e4m3fn, 0),
                "weight_scale": (shape, torch.float32, 1)}

    @classmethod
    def from_dense(cls, linear: nn.Linear, *, granularity: str = "per_channel", block: int = 128,
                   **_: Any) -> KernelFp8Linear:
        mod = cls(linear.in_features, linear.out_features, linear.bias is not None, linear.weight.dtype,
                  linear.weight.device, granularity=granularity, block=block)
        q, s = quantize_weight_fp8(linear.weight.detach(), granularity, block)
        mod._fill({"weight_fp8": q, "weight_scale": s}, None)
        if linear.bias is not None:
            with torch.no_grad():
                mod.bias.copy_(linear.bias.detach())
        return mod

    def dequantize(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        """``codes * scale`` as a dense ``[N, K]`` weight (scales broadcast per tensor, channel or block)."""
        n, k = self.out_features, self.in_features
        s = self.weight_scale.float()
        if self.granularity == "block2d":
            s = s.repeat_interleave(self.block, 0).repeat_interleave(self.block, 1)[:n, :k]
        else:
            s = s.reshape(-1, 1)
        return (self.weight_fp8.float() * s).to(dtype or torch.float32)

    def quant_spec(self) -> dict[str, Any]:
        return {"granularity": self.granularity, "block": self.block}

    def _linear(self, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        return fp8_linear(x, self.weight_fp8, self.weight_scale, bias, block=self.block)


class KernelInt8Linear(_PackedLinear):
    """INT8 W8A8: per-channel weight scales, per-token activation scales computed on the fly (buffers
    ``weight_int8`` and ``weight_scale``)."""

    kind: ClassVar[str] = "int8"

    def _buffer_specs(self, dtype: torch.dtype | None) -> _Buffers:
        return {"weight_int8": ((self.out_features, self.in_features), torch.int8, 0),
                "weight_scale": ((self.out_features,), torch.float32, 1)}

    @classmethod
    def from_dense(cls, linear: nn.Linear, **_: Any) -> KernelInt8Linear:
        mod = cls(linear.in_features, linear.out_features, linear.bias is not None, linear.weight.dtype,
                  linear.weight.device)
        q, s = quantize_weight_int8(linear.weight.detach())  # one scale per output channel = per row of W
        mod._fill({"weight_int8": q, "weight_scale": s}, None)
        if linear.bias is not None:
            with torch.no_grad():
                mod.bias.copy_(linear.bias.detach())
        return mod

    def dequantize(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        return (self.weight_int8.float() * self.weight_scale.float().reshape(-1, 1)).to(dtype or torch.float32)

    def _linear(self, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        return int8_linear(x, self.weight_int8, self.weight_scale, bias)


PACKED_LINEAR_CLASSES: dict[str, type] = {"w4a16": KernelW4A16Linear, "w8a16": KernelW8A16Linear,
                                          "fp8": KernelFp8Linear, "int8": KernelInt8Linear}
_PACKED_TYPES = {KernelW4A16Linear: PackedW4, KernelW8A16Linear: PackedW8}


def make_packed_linear(kind: str, linear: nn.Linear | None = None, *, packed: PackedW4 | PackedW8 | None = None,
                       bias: torch.Tensor | None = None, in_features: int | None = None,
                       out_features: int | None = None, **kw: Any) -> nn.Module:
    """A kernel-backed packed linear of ``kind`` (GEMM-family kinds of ``forge/kernels/ops_gemm.py:1025-1068``): from
    packed data, from a dense ``nn.Linear``, or empty by shape (to be filled by ``load_state_dict``)."""
    if kind not in PACKED_LINEAR_CLASSES:
        raise ConfigError(f"unknown packed linear kind {kind!r}: use one of {sorted(PACKED_LINEAR_CLASSES)}")
    cls = PACKED_LINEAR_CLASSES[kind]
    if packed is not None:
        if _PACKED_TYPES.get(cls) is not type(packed):
            raise ConfigError(f"{type(packed).__name__} cannot back a {kind!r} linear")
        return cls.from_packed(packed, bias)
    if linear is not None:
        return cls.from_dense(linear, **kw)
    if in_features is None or out_features is None:
        raise ConfigError("make_packed_linear needs a dense `linear`, `packed` data, or in_features / out_features")
    return cls.from_shape(in_features, out_features, bias is not None, **kw)


__all__ = [
    "KernelFp8Linear", "KernelInt8Linear", "KernelW4A16Linear", "KernelW8A16Linear", "PACKED_LINEAR_CLASSES",
    "device_selftest", "force_ref", "forced_impl", "fp8_linear", "int8_gemm", "int8_linear", "kernel_debug",
    "kernel_strict", "last_kernel", "last_path", "make_packed_linear", "prepare_fp8_scales", "prepare_w4", "prepare_w4_sz8", "quantize_act_fp8",
    "quantize_act_int8", "quantize_weight_fp8", "quantize_weight_int8", "reset_failure_memo", "w4_dequant", "w4a16_linear", "w8a16_linear",
]
