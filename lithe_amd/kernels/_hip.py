"""ctypes boundary to ``liblithe_amd.so`` (the gfx950 HIP kernels behind ``include/lithe_amd.h``).

This module replaces the reference's optional-Triton dispatch
(``lithe/kernels/_triton.py:1-18``): GPU tensors always go to the HIP library,
and there is no CPU fallback. Every public entry point of ``lithe_amd`` that
computes raises ``RuntimeError`` when the library is not built or a tensor is
not on a GPU.

torch is imported first so that its bundled ROCm runtime (``libamdhip64.so.7``)
is the one the library binds to: one HIP runtime, one set of streams.
"""
from __future__ import annotations

import ctypes
import os
import threading
import weakref
from typing import Dict, Optional, Tuple

import numpy as np
import torch

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG, "_lib", "liblithe_amd.so")

# ------------------------------------------------------------------ C constants (lithe_amd.h)
OK = 0
ERR_NULL, ERR_SHAPE, ERR_ALIGN, ERR_DTYPE, ERR_RANGE, ERR_WORKSPACE, ERR_HIP, ERR_LEVELS, ERR_UNSUPPORTED = (
    -1, -2, -3, -4, -5, -6, -7, -8, -9)
ERR_OVERLAP = -10
DT_BF16, DT_F32, DT_F16, DT_I16, DT_I32, DT_I64, DT_U16 = 1, 2, 3, 4, 5, 6, 7
STATIC_SCRATCH_BYTES = 16777216
IDX_PACKED9, IDX_LEVEL_I32, IDX_LEVEL_I16, IDX_BLOCK_I16 = 1, 2, 3, 4
FACTOR_INDEXED, FACTOR_DENSE = 1, 2

_TORCH_DT = {torch.bfloat16: DT_BF16, torch.float32: DT_F32, torch.float16: DT_F16,
             torch.int16: DT_I16, torch.int32: DT_I32, torch.int64: DT_I64}


class IndexSrc(ctypes.Structure):
    _fields_ = [("base", ctypes.c_void_p), ("kind", ctypes.c_int32), ("num_levels", ctypes.c_int32),
                ("slot_stride", ctypes.c_int64), ("level_stride", ctypes.c_int64),
                ("block_off", ctypes.c_int64), ("n_slots", ctypes.c_int64)]


class Lut(ctypes.Structure):
    _fields_ = [("num_levels", ctypes.c_int32), ("value", (ctypes.c_float * 10) * 4)]


class Factors(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("dense_dtype", ctypes.c_int32),
                ("a_idx", IndexSrc), ("b_idx", IndexSrc), ("lut_a", Lut), ("lut_b", Lut),
                ("dense_a", ctypes.c_void_p), ("dense_b", ctypes.c_void_p), ("n_dense", ctypes.c_int64)]


class Routes(ctypes.Structure):
    _fields_ = [("slot", ctypes.c_void_p), ("weight_sqrt", ctypes.c_void_p),
                ("slot_scale", ctypes.c_void_p), ("n_route", ctypes.c_int32)]


class Module(ctypes.Structure):
    _fields_ = [("x", ctypes.c_void_p), ("y", ctypes.c_void_p), ("seq", ctypes.c_int64), ("d_in", ctypes.c_int64),
                ("d_out", ctypes.c_int64), ("a_block_off", ctypes.c_int64), ("b_block_off", ctypes.c_int64),
                ("out_scale", ctypes.c_float)]


MAX_GROUP_MODULES = 8


# Every symbol include/lithe_amd.h declares, with its ctypes signature.
_P, _I32, _I64, _F32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
SIGNATURES = {
    "lithe_abi_version": ([], _I32),
    "lithe_status_string": ([_I32], ctypes.c_char_p),
    "lithe_pack9_host": ([_P, _I64, _P], _I32),
    "lithe_pack9": ([_P, _I32, _I64, _P, _P, _P], _I32),
    "lithe_unpack9": ([_P, _I64, _P, _I32, _P], _I32),
    "lithe_decode": ([ctypes.POINTER(IndexSrc), _P, _I32, _I64, _P, ctypes.POINTER(Lut),
                      ctypes.POINTER(Lut), _P, _I32, _I64, _P, _P], _I32),
    "lithe_lora_workspace_bytes": ([_I64, _I64, _I64, _I64, _I32, _I32, _I32], _I64),
    "lithe_lora_delta": ([_P, _I32, _I64, _I64, _I64, _P, _I32, _I64, _I32, _I32,
                          ctypes.POINTER(Factors), ctypes.POINTER(Routes), _P, _F32, _P,
                          _P, _I64, _P], _I32),
    "lithe_lora_delta_noalloc": ([_P, _I32, _I64, _I64, _I64, _P, _I32, _I64, _I32, _I32,
                                  ctypes.POINTER(Factors), ctypes.POINTER(Routes), _P, _F32, _P, _P, _P], _I32),
    "lithe_lora_delta_shared_x": ([_P, _I32, _I64, _I64, _I64, _I32, _P, _I32, _P, _I32, _I32,
                                   ctypes.POINTER(Factors), ctypes.POINTER(Routes), _P, _P, _P, _I64, _P], _I32),
    "lithe_workspace_errors": ([_P, _P, _I32, _P], _I32),
    "lithe_lora_grouped_workspace_bytes": ([_I64, _I32, _P, _I32, _I32, _I32], _I64),
    "lithe_lora_delta_grouped": ([_I32, _P, _I32, _I32, _I64, _I32, _I32, ctypes.POINTER(Factors),
                                  ctypes.POINTER(Routes), _P, _I64, _P], _I32),
    "lithe_decode_stacked": ([ctypes.POINTER(IndexSrc), _P, _I32, _I64, _I32, _P, _P, ctypes.POINTER(Lut),
                              ctypes.POINTER(Lut), _P, _I32, _P, _P], _I32),
    "lithe_encode": ([_P, _I64, _P, ctypes.POINTER(Lut), ctypes.POINTER(Lut), _P, _I32, _I64, _I64, _P, _P], _I32),
    "lithe_ingest_table": ([_I32, _P, _P, _I32, _P], _I32),
    "lithe_ingest_host": ([_P, _I64, _I32, _I32, _P, _P, _I64], _I32),
    "lithe_ingest": ([_P, _I64, _I32, _I32, _P, _P, _I64, _P, _P], _I32),
}

_lib = None
_lib_err: Optional[str] = None
_lock = threading.Lock()


def load(path: str = LIB_PATH):
    """Load the HIP library (once). Raises RuntimeError when it is missing."""
    global _lib, _lib_err
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(path):
                _lib_err = f"{path} is not built (run __graft_entry__.build() or python -m lithe_amd.csrc.build)"
                raise RuntimeError(_lib_err)
            lib = ctypes.CDLL(path)
            for name, (args, res) in SIGNATURES.items():
                try:
                    fn = getattr(lib, name)
                except AttributeError:
                    _lib_err = f"{path} is stale: it does not export {name} (rebuild it)"
                    raise RuntimeError(_lib_err) from None
                fn.argtypes = args
                fn.restype = res
            _lib = lib
    return _lib


def library_available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


def gpu_available() -> bool:
    return library_available() and torch.cuda.is_available()


# Mirrors the role of HAS_TRITON (lithe/kernels/_triton.py:6-13): the HIP path can run.
HAS_HIP = library_available()


def status_string(code: int) -> str:
    return load().lithe_status_string(code).decode()


def check(code: int, what: str) -> None:
    if code == OK:
        return
    msg = f"{what}: {status_string(code)} (status {code})"
    if code in (ERR_HIP,):
        raise RuntimeError(msg)
    raise ValueError(msg)


def require_gpu(*tensors: torch.Tensor) -> None:
    """Fail loudly unless the library is loaded and every tensor is on a GPU."""
    load()
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("lithe_amd kernels run on the GPU only (HIP, gfx950); got a tensor on "
                               f"{t.device}. Move the inputs to a cuda device.")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_DT[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


# ------------------------------------------------------------------ value tables from pools
def _popcount_classes(block_size: int, n_bits: int) -> np.ndarray:
    """P[k, t] = popcount((k ^ m_t) & (2**n_bits - 1)), the codeword coordinate class."""
    t = np.arange(block_size, dtype=np.uint32)
    q = np.arange(n_bits, dtype=np.uint32)
    bits = (np.bitwise_count(t[:, None] & q[None, :]) & 1) ^ 1           # (block, n_bits)
    masks = (bits.astype(np.uint32) << q[None, :]).sum(axis=1).astype(np.uint32)
    k = np.arange(1 << n_bits, dtype=np.uint32)
    return np.bitwise_count((k[:, None] ^ masks[None, :]) & np.uint32((1 << n_bits) - 1)).astype(np.int64)


_CLASSES = _popcount_classes(64, 9)
# id(pool tensor) -> {(version, source dtype, target dtype): Lut}. A finalizer drops the
# entry when the tensor dies, so a later tensor that reuses the id (or the memory)
# can never see a stale table.
_lut_cache: Dict[int, Dict[Tuple, Lut]] = {}


def version_of(t: torch.Tensor):
    """The tensor's version counter, or None for an inference tensor (``torch.inference_mode``
    tensors keep none; they cannot be written outside inference mode)."""
    return None if t.is_inference() else t._version


def lut_from_pools(pools: torch.Tensor, dtype: Optional[torch.dtype] = None) -> Lut:
    """Value table of a (L, 512, 64) pool stack after casting it to ``dtype``.

    The pools must be the twin Hadamard pools (any per-level scale): every entry
    pools[l, k, t] must equal a per-level function of popcount((k ^ m_t) & 511).
    This is checked bit for bit; other pools raise ValueError.
    """
    if pools.dim() != 3 or tuple(pools.shape[1:]) != (512, 64):
        raise ValueError("lithe_amd decodes the 9-bit, 64-wide codebook: pools must be (L, 512, 64)")
    L = int(pools.shape[0])
    if not 1 <= L <= 4:
        raise ValueError("num_levels must be in [1, 4]")
    dtype = dtype or pools.dtype
    key = (version_of(pools), pools.dtype, dtype)
    per = _lut_cache.get(id(pools))
    if per is not None and key in per:
        return per[key]
    host = pools.detach().to(dtype).to("cpu", torch.float32).numpy()
    lut = Lut()
    lut.num_levels = L
    for level in range(L):
        vals = np.zeros(10, dtype=np.float32)
        for p in range(10):
            sel = host[level][_CLASSES == p]
            vals[p] = sel[0]
        expanded = vals[_CLASSES]
        if not np.array_equal(expanded.view(np.uint32), host[level].view(np.uint32)):
            raise ValueError("pools are not twin Hadamard codebook pools (lithe_amd regenerates codewords "
                             "from their closed form and cannot decode arbitrary pools)")
        for p in range(10):
            lut.value[level][p] = float(vals[p])
    if per is None:
        per = {}
        _lut_cache[id(pools)] = per
        weakref.finalize(pools, _lut_cache.pop, id(pools), None)
    per[key] = lut
    return lut


# ------------------------------------------------------------------ workspaces
_workspaces: Dict[Tuple[int, int], torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Zero-initialised scratch for lithe_lora_delta, one per (device, stream), grown on demand.
    A grown workspace starts with the error word of the one it replaces (copied on the same
    stream), so errors recorded before the growth are still reported."""
    dev = torch.device(device)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(dev).cuda_stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(int(nbytes), 1 << 20)
        if ws is not None:
            size = max(size, 2 * ws.numel())
        grown = torch.zeros(size, dtype=torch.uint8, device=dev)
        if ws is not None:
            grown[:4].copy_(ws[:4])
        ws = grown
        _workspaces[key] = ws
    return ws


def workspace_errors(device: Optional[torch.device] = None, clear: bool = True) -> int:
    """Error bits recorded in-kernel since the last clear (1: bad slot id, 2: index > 511)."""
    flags = 0
    for (dev_idx, stream), ws in list(_workspaces.items()):
        if device is not None and torch.device(device).index not in (None, dev_idx):
            continue
        out = ctypes.c_int32(0)
        check(load().lithe_workspace_errors(ptr(ws), ctypes.byref(out), int(clear), ctypes.c_void_p(stream)),
              "lithe_workspace_errors")
        flags |= out.value
    return flags
