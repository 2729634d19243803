"""ctypes binding of the C restatement ``oracle/c/lithe_oracle.c`` (test infrastructure only).

``build()`` runs the Makefile next to this file; ``lib()`` loads the result.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "liblithe_oracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-B", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        _lib.lo_pack9.argtypes = [p, i64, p]
        _lib.lo_pack9.restype = ctypes.c_int
        _lib.lo_unpack9.argtypes = [p, i64, p]
        _lib.lo_bf16.argtypes = [p, p, i64]
        _lib.lo_decode.argtypes = [p, i64, ctypes.c_int, p, p, p, p, p]
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def pack(indices) -> np.ndarray:
    idx = np.ascontiguousarray(np.asarray(indices).reshape(-1), dtype=np.uint16)
    words = np.zeros(-(-idx.size // 7), dtype=np.uint64)
    if lib().lo_pack9(_ptr(idx), idx.size, _ptr(words)) != 0:
        raise ValueError("indices must be < 512 for 9-bit packing")
    return words


def unpack(words, n: int) -> np.ndarray:
    w = np.ascontiguousarray(words, dtype=np.uint64)
    out = np.empty(n, dtype=np.int64)
    lib().lo_unpack9(_ptr(w), n, _ptr(out))
    return out


def bf16_bits(x) -> np.ndarray:
    f = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().lo_bf16(_ptr(f), _ptr(out), f.size)
    return out


def decode(words, n_blocks: int, levels: int, sides, pool_a, pool_b, want="f32"):
    """(n_blocks, 64) decode of a packed stream; ``want`` "f32" or "bf16" (uint16 bits)."""
    w = np.ascontiguousarray(words, dtype=np.uint64)
    s = None if sides is None else np.ascontiguousarray(sides, dtype=np.int8)
    pa = np.ascontiguousarray(pool_a, dtype=np.float32)
    pb = np.ascontiguousarray(pool_b, dtype=np.float32)
    f32 = np.empty((n_blocks, 64), np.float32) if want == "f32" else None
    b16 = np.empty((n_blocks, 64), np.uint16) if want == "bf16" else None
    lib().lo_decode(_ptr(w), n_blocks, levels, _ptr(s), _ptr(pa), _ptr(pb), _ptr(f32), _ptr(b16))
    return f32 if want == "f32" else b16
