"""Build and load the C oracle (``oracle/c/oracle.c``) -- test infrastructure only.

``build()`` compiles it with gcc into ``oracle/_lib/liboracle.so`` (git-ignored, travels to the GPU box with the tree).
``load()`` returns thin numpy wrappers.  Recipe: ``gcc -O2 -ffp-contract=off -fPIC -shared oracle/c/oracle.c``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "c", "oracle.c")
OUT_DIR = os.path.join(HERE, "_lib")
LIB = os.path.join(OUT_DIR, "liboracle.so")


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = LIB + f".tmp{os.getpid()}"
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-o", tmp, SRC]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        lib = ctypes.CDLL(LIB)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.fgo_w4_dequant_f32.argtypes = [P, I64, P, I64, P, I64, P, I, I64, I64, P]
        lib.fgo_w4a16_gemm_f32.argtypes = [P, I64, I64, P, I64, P, I64, P, I64, P, I, I64, P, P]
        lib.fgo_int8_gemm_i32.argtypes = [P, I64, I64, P, I64, P]
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _packed_args(packed: dict):
    qw = np.ascontiguousarray(packed["qweight"], dtype=np.int32)
    sc = np.ascontiguousarray(packed["scales"], dtype=np.float32)
    zr = None if packed["zeros"] is None else np.ascontiguousarray(packed["zeros"], dtype=np.int32)
    gi = None if packed["g_idx"] is None else np.ascontiguousarray(packed["g_idx"], dtype=np.int32)
    k = packed["k"]
    gs = k if packed["group_size"] <= 0 else packed["group_size"]
    return qw, sc, zr, gi, gs


def w4_dequant(packed: dict) -> np.ndarray:
    qw, sc, zr, gi, gs = _packed_args(packed)
    n, k = packed["n"], packed["k"]
    out = np.empty((n, k), dtype=np.float32)
    _load().fgo_w4_dequant_f32(_p(qw), qw.shape[1], _p(sc), sc.shape[1], _p(zr), 0 if zr is None else zr.shape[1],
                               _p(gi), gs, n, k, _p(out))
    return out


def w4a16_gemm(x: np.ndarray, packed: dict, bias: np.ndarray | None = None) -> np.ndarray:
    qw, sc, zr, gi, gs = _packed_args(packed)
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    n = packed["n"]
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y = np.empty((m, n), dtype=np.float32)
    _load().fgo_w4a16_gemm_f32(_p(x), m, k, _p(qw), qw.shape[1], _p(sc), sc.shape[1], _p(zr),
                               0 if zr is None else zr.shape[1], _p(gi), gs, n, _p(b), _p(y))
    return y


def int8_gemm_i32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    m, k = a.shape
    n = b.shape[0]
    c = np.empty((m, n), dtype=np.int32)
    _load().fgo_int8_gemm_i32(_p(a), m, k, _p(b), n, _p(c))
    return c
