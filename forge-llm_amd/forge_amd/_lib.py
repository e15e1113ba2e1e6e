"""ctypes binding of libforge_mi355x.so (declarations: include/forge_mi355x.h).

There is no fallback: if the library is missing or fails to load, every op raises :class:`HipExtensionMissing`.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

from .errors import ForgeError, HardwareUnsupported

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libforge_mi355x.so")

# element type codes (FG_* in forge_mi355x.h)
F32, F16, BF16, E4M3, I8, I32 = 0, 1, 2, 3, 4, 5
DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.float8_e4m3fn: E4M3,
              torch.int8: I8, torch.int32: I32}
W4A16_SCRATCH_BYTES = 64 << 20  # FG_W4A16_SCRATCH_BYTES
# status codes
OK, EINVAL, EUNSUPPORTED, EHIP = 0, 1, 2, 3
# W4A16 impl codes
W4_AUTO, W4_GEMV, W4_MFMA, W4_GENERIC, W4_PREFILL, W4_DEQUANT_GEMM = 0, 1, 2, 3, 4, 5
W4_IMPL = {None: W4_AUTO, "auto": W4_AUTO, "gemv": W4_GEMV, "mfma": W4_MFMA, "generic": W4_GENERIC,
           "prefill": W4_PREFILL, "dequant_gemm": W4_DEQUANT_GEMM}
GEMV_AUTO, GEMV_SPLIT, GEMV_TILE, GEMV_WAVE = 0, 1, 2, 3
GEMV_KERNEL = {None: GEMV_AUTO, "auto": GEMV_AUTO, "split": GEMV_SPLIT, "tile": GEMV_TILE, "wave": GEMV_WAVE}


class HipExtensionMissing(ForgeError):
    """libforge_mi355x.so is not built or cannot be loaded (run ``python __graft_entry__.py`` / ``forge_amd.build``)."""

    code = "hip_extension_missing"


class KernelLaunchError(ForgeError):
    """A C-ABI entry point returned a non-zero status."""

    code = "kernel_launch_error"

    def __init__(self, message: str = "", *, status: int = -1) -> None:
        super().__init__(message, details={"status": status})
        self.status = status


class W4Config(ctypes.Structure):
    _fields_ = [("impl", ctypes.c_int32), ("rows_per_wave", ctypes.c_int32), ("max_blocks", ctypes.c_int32),
                ("tile_m", ctypes.c_int32), ("split_k", ctypes.c_int32), ("tile_n", ctypes.c_int32),
                ("gemv_kernel", ctypes.c_int32), ("reserved", ctypes.c_int32 * 1)]


class MMConfig(ctypes.Structure):
    _fields_ = [("tile_m", ctypes.c_int32), ("tile_n", ctypes.c_int32), ("reserved", ctypes.c_int32 * 6)]


P, I64, I32_, INT, SZ, F32_ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int, ctypes.c_size_t, ctypes.c_float

SIGNATURES = {
    "fg_w4a16_gemm": ([P, I64, INT, P, I64, P, INT, I64, P, I64, P, P, P, INT, P, I64, I64, I64, I64, I32_, I32_,
                       ctypes.POINTER(W4Config), P, SZ, P], INT),
    "fg_w4a16_gemm_noalloc": ([P, I64, INT, P, I64, P, INT, I64, P, I64, P, P, P, INT, P, I64, I64, I64, I64, I32_,
                               I32_, ctypes.POINTER(W4Config), P], INT),
    "fg_w4a16_gemm_cdna4": ([P, I64, INT, P, I64, P, INT, I64, P, I64, P, INT, P, I64, I64, I64, I64, I32_, I32_, P,
                             SZ, P], INT),
    "fg_w4a16_cdna4_workspace_bytes": ([I64, I64, I64, I32_], SZ),
    "fg_w4a16_gemv_sz8": ([P, I64, INT, P, I64, P, INT, P, P, INT, P, I64, I64, I64, I64, I32_, I32_, P], INT),
    "fg_w4a16_workspace_bytes": ([I64, I64, I64, I32_, I32_, I32_, I32_, ctypes.POINTER(W4Config)], SZ),
    "fg_w4_dequant": ([P, I64, P, INT, I64, P, I64, P, P, INT, I64, I64, I64, I32_, I32_, P], INT),
    "fg_w8a16_gemm": ([P, I64, INT, P, I64, P, INT, I64, P, INT, P, I64, I64, I64, I64, I32_, I32_,
                       ctypes.POINTER(W4Config), P, SZ, P], INT),
    "fg_w8a16_workspace_bytes": ([I64, I64, I64, I32_, ctypes.POINTER(W4Config)], SZ),
    "fg_int8_gemm": ([P, I64, P, I64, P, I64, P, I64, P, INT, P, I64, INT, I64, I64, I64, ctypes.POINTER(MMConfig), P],
                     INT),
    "fg_fp8_gemm": ([P, I64, P, I64, I64, P, I64, P, I64, I64, I32_, I32_, I32_, P, INT, P, I64, INT, I64, I64, I64,
                     ctypes.POINTER(MMConfig), P], INT),
    "fg_quant_int8_rowwise": ([P, I64, INT, P, I64, P, I64, I64, P], INT),
    "fg_quant_fp8_rowwise": ([P, I64, INT, P, I64, P, I64, I64, P, P, INT, F32_, I32_, P], INT),
    "fg_quant_fp8_block": ([P, I64, INT, P, I64, P, I64, I64, I64, I32_, I32_, P, P], INT),
    "fg_version": ([], ctypes.c_char_p),
    "fg_last_error": ([], ctypes.c_char_p),
    "fg_last_kernel": ([], ctypes.c_char_p),
    "fg_device_ok": ([INT], INT),
}

_LIB = None
_LOCK = threading.Lock()
_DEVICE_OK: dict[int, bool] = {}


def lib():
    """The loaded library (raises :class:`HipExtensionMissing` when it is not built)."""
    global _LIB
    if _LIB is None:
        with _LOCK:
            if _LIB is None:
                if not os.path.exists(LIB_PATH):
                    raise HipExtensionMissing(f"{LIB_PATH} is not built; run `python __graft_entry__.py build` "
                                              "(hipcc --offload-arch=gfx950) first")
                try:
                    handle = ctypes.CDLL(LIB_PATH)
                except OSError as e:
                    raise HipExtensionMissing(f"cannot load {LIB_PATH}: {e}") from e
                for name, (args, res) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.argtypes = args
                    fn.restype = res
                _LIB = handle
    return _LIB


def last_error() -> str:
    return (lib().fg_last_error() or b"").decode()


def last_kernel() -> str:
    """The kernel (and launch form) the calling thread's last launch ran, as the library recorded it."""
    return (lib().fg_last_kernel() or b"").decode()


def check(status: int, what: str) -> None:
    if status != OK:
        raise KernelLaunchError(f"{what} failed (status {status}): {last_error()}", status=status)


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_device(t: torch.Tensor, op: str) -> None:
    """Raise unless ``t`` lives on a gfx950 GPU this library can run on (checked once per device)."""
    if not t.is_cuda:
        raise HardwareUnsupported(f"{op}: forge_amd runs on MI355X (gfx950) GPUs only; got a {t.device.type} tensor "
                                  "(there is no CPU path in this build)")
    idx = t.device.index if t.device.index is not None else torch.cuda.current_device()
    ok = _DEVICE_OK.get(idx)
    if ok is None:
        ok = _DEVICE_OK[idx] = bool(lib().fg_device_ok(idx))
    if not ok:
        raise HardwareUnsupported(f"{op}: {last_error()}")


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dt]
    except KeyError:
        raise HardwareUnsupported(f"dtype {dt} is not supported by forge_amd kernels") from None
