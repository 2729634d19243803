"""Internal driver of ``lithe_lora_delta``: builds the C descriptors and launches.

All per-sample LoRA entry points (index-resident, packed-bank, dense-factor,
serve.py routing, LitheLinear) funnel through :func:`lora_delta`.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _hip


def index_source(idx: torch.Tensor, levels: int, n_blocks: int) -> _hip.IndexSrc:
    """Descriptor of a level-major (n_slots, L, n_blocks) int32 / int16 index tensor."""
    if idx.dim() != 3 or idx.shape[1] != levels or idx.shape[2] != n_blocks:
        raise ValueError("index pools must be (n_slots, L, n_blocks)")
    if idx.dtype not in (torch.int32, torch.int16):
        raise ValueError(f"index tensors must be int32 or int16, got {idx.dtype}")
    if idx.stride(2) != 1:
        raise ValueError("index tensors must be contiguous along the block dimension")
    s = _hip.IndexSrc()
    s.base = idx.data_ptr()
    s.kind = _hip.IDX_LEVEL_I32 if idx.dtype == torch.int32 else _hip.IDX_LEVEL_I16
    s.num_levels = levels
    s.slot_stride = idx.stride(0)
    s.level_stride = idx.stride(1)
    s.block_off = 0
    s.n_slots = idx.shape[0]
    return s


def packed_source(words: torch.Tensor, levels: int, block_off: int) -> _hip.IndexSrc:
    """Descriptor of a packed bank (n_slots, n_words) uint64 (or one slot, (n_words,))."""
    w = words if words.dim() == 2 else words.view(1, -1)
    if w.stride(1) != 1:
        raise ValueError("packed words must be contiguous")
    s = _hip.IndexSrc()
    s.base = w.data_ptr()
    s.kind = _hip.IDX_PACKED9
    s.num_levels = levels
    s.slot_stride = w.stride(0) if w.shape[0] > 1 else w.shape[1]
    s.level_stride = 0
    s.block_off = int(block_off)
    s.n_slots = w.shape[0]
    return s


def indexed_factors(a_src: _hip.IndexSrc, b_src: _hip.IndexSrc, lut_a: _hip.Lut, lut_b: _hip.Lut) -> _hip.Factors:
    f = _hip.Factors()
    f.kind = _hip.FACTOR_INDEXED
    f.a_idx = a_src
    f.b_idx = b_src
    f.lut_a = lut_a
    f.lut_b = lut_b
    return f


def dense_factors(a: torch.Tensor, b: torch.Tensor) -> _hip.Factors:
    f = _hip.Factors()
    f.kind = _hip.FACTOR_DENSE
    f.dense_dtype = _hip.dtype_code(a.dtype)
    f.dense_a = a.data_ptr()
    f.dense_b = b.data_ptr()
    f.n_dense = a.shape[0]
    return f


def routes(slot: torch.Tensor, weight_sqrt: Optional[torch.Tensor] = None,
           slot_scale: Optional[torch.Tensor] = None) -> _hip.Routes:
    """slot (n_batch, n_route) int32 on the GPU; weight_sqrt same shape fp32; slot_scale (n_slots,) fp32."""
    r = _hip.Routes()
    r.slot = slot.data_ptr()
    r.weight_sqrt = weight_sqrt.data_ptr() if weight_sqrt is not None else None
    r.slot_scale = slot_scale.data_ptr() if slot_scale is not None else None
    r.n_route = slot.shape[1] if slot.dim() == 2 else 1
    return r


_need: dict = {}    # workspace bytes per (n_batch, seq, d_in, d_out, rank, n_route, x dtype)


def lora_delta(x: torch.Tensor, y: torch.Tensor, *, rank: int, factors: _hip.Factors, route: _hip.Routes,
               accumulate: bool, mid_scale: Optional[torch.Tensor] = None, out_scale: float = 1.0,
               out_scale_vec: Optional[torch.Tensor] = None, keep: tuple = ()) -> torch.Tensor:
    """y (B, M, d_out) <- per-sample delta of x (B, M, d_in); see lithe_lora_delta in lithe_amd.h.

    ``keep`` holds tensors whose memory the descriptors point at, so that they
    outlive the enqueue.
    """
    lib = _hip.load()
    n_batch, seq, d_in = x.shape
    d_out = y.shape[2]
    xd = _hip.dtype_code(x.dtype)
    wkey = (n_batch, seq, d_in, d_out, rank, route.n_route, xd)
    need = _need.get(wkey)
    if need is None:
        need = lib.lithe_lora_workspace_bytes(n_batch, seq, d_in, d_out, rank, route.n_route, xd)
        _hip.check(int(need) if need < 0 else 0, "lithe_lora_workspace_bytes")
        if len(_need) > 4096:
            _need.clear()
        _need[wkey] = need
    ws = _hip.workspace(x.device, int(need))
    rc = lib.lithe_lora_delta(
        _hip.ptr(x), xd, n_batch, seq, d_in, _hip.ptr(y), _hip.dtype_code(y.dtype), d_out,
        int(bool(accumulate)), int(rank), ctypes.byref(factors), ctypes.byref(route),
        _hip.ptr(mid_scale), ctypes.c_float(float(out_scale)), _hip.ptr(out_scale_vec),
        _hip.ptr(ws), ws.numel(), _hip.stream_of(x.device))
    _hip.check(rc, "lithe_lora_delta")
    return y
