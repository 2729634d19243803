"""Blocking and the residual decode of the twin Hadamard codebook.

API of ``lithe/quant.py:23-43, 74-92`` (the decode half). A factor of any shape
is flattened row-major, zero-padded to a multiple of the 64-value block and
viewed as (n_blocks, 64). ``rvq_decode_blocks`` runs on the GPU through
``lithe_decode``: the L levels are summed in fp32 in level order, the same
order as the reference, so the result is bit-identical. The encode half
(search, STE) belongs to training and is not part of this library.
"""
from __future__ import annotations

import ctypes

import torch

from . import codebook as cb
from .kernels import _hip


def blockify(w: torch.Tensor, block_size: int = cb.BLOCK_SIZE) -> torch.Tensor:
    """Flatten ``w`` row-major and reshape to (n_blocks, block_size) with zero padding."""
    flat = w.reshape(-1)
    pad = (-flat.numel()) % block_size
    if pad:
        flat = torch.cat([flat, flat.new_zeros(pad)])
    return flat.view(-1, block_size)


def unblockify(blocks: torch.Tensor, shape) -> torch.Tensor:
    n = 1
    for s in shape:
        n *= int(s)
    return blocks.reshape(-1)[:n].view(*[int(s) for s in shape])


def num_blocks(shape, block_size: int = cb.BLOCK_SIZE) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return -(-n // block_size)


def rvq_decode_blocks(indices: torch.Tensor, pools: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Sum of selected codewords: indices (L, N) -> (N, 64) in ``dtype`` (fp32 by default), on the GPU."""
    _hip.require_gpu(indices)
    if indices.dim() != 2 or indices.shape[0] != pools.shape[0]:
        raise ValueError("indices must be (L, N) with L = pools.shape[0]")
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("decode output must be float32 or bfloat16")
    L, n = int(indices.shape[0]), int(indices.shape[1])
    idx = indices if indices.dtype in (torch.int32, torch.int16) else indices.to(torch.int32)
    idx = idx.contiguous()
    lut = _hip.lut_from_pools(pools, torch.float32)
    out = torch.empty((n, cb.BLOCK_SIZE), dtype=dtype, device=indices.device)
    if n == 0:
        return out
    src = _hip.IndexSrc()
    src.base = idx.data_ptr()
    src.kind = _hip.IDX_LEVEL_I32 if idx.dtype == torch.int32 else _hip.IDX_LEVEL_I16
    src.num_levels = L
    src.slot_stride = L * n
    src.level_stride = n
    src.block_off = 0
    src.n_slots = 1
    rc = _hip.load().lithe_decode(ctypes.byref(src), None, 1, n, None, ctypes.byref(lut), None,
                                  _hip.ptr(out), _hip.dtype_code(dtype), n * cb.BLOCK_SIZE, None,
                                  _hip.stream_of(indices.device))
    _hip.check(rc, "lithe_decode")
    return out


def decode(indices: torch.Tensor, shape, pools: torch.Tensor) -> torch.Tensor:
    """fp32 factor of ``shape`` decoded from (L, n_blocks) indices."""
    return unblockify(rvq_decode_blocks(indices, pools), shape)
