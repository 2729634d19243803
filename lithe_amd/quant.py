"""Blocking, the residual decode and the greedy residual encode of the twin Hadamard codebook.

API of ``lithe/quant.py:23-92``. A factor of any shape is flattened row-major,
zero-padded to a multiple of the 64-value block and viewed as (n_blocks, 64).
``rvq_decode_blocks`` runs on the GPU through ``lithe_decode``: the L levels are
summed in fp32 in level order, the same order as the reference, so the result is
bit-identical. ``nearest_index`` / ``rvq_encode_blocks`` / ``encode`` run on the
GPU through ``lithe_encode`` (the closed-form search: bit q of a level's index is
set exactly when the residual's projection on Hadamard column q is positive). The
straight-through estimator (``ste``) belongs to training and is not part of this
library.
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


_UNIT_POOL = {}     # device -> (1, 512, 64) unit-scale pool (a level's scale does not move the argmin)


def nearest_index(x: torch.Tensor, proj: torch.Tensor) -> torch.Tensor:
    """Index (N,) int64 of the nearest codeword of every 64-value block of ``x`` (N, 64)
    (``lithe/quant.py:46-51``); ``proj`` must be the codebook's Hadamard generator. Every
    codeword of a level has one norm, so the index does not depend on the level's scale."""
    from .kernels import search
    search._check_proj(proj, x.shape[-1])
    key = str(x.device)
    if key not in _UNIT_POOL:
        _UNIT_POOL[key] = cb.build_pools([1.0], x.shape[-1]).to(x.device)
    idx, _ = search._encode(x, _UNIT_POOL[key], want_recon=False)
    return idx[0]


def rvq_encode_blocks(blocks: torch.Tensor, pools: torch.Tensor,
                      proj: torch.Tensor) -> "tuple[torch.Tensor, torch.Tensor]":
    """Greedy residual encode: (indices (L, N) int64, reconstruction (N, 64) fp32)
    (``lithe/quant.py:54-71``), all levels in one launch."""
    from .kernels import search
    return search.rvq_encode_blocks_fast(blocks, pools, proj)


def encode(w: torch.Tensor, pools: torch.Tensor, proj: torch.Tensor) -> "tuple[torch.Tensor, torch.Tensor]":
    """Quantise a factor of any shape: (indices (L, n_blocks) int64, w_hat with w's shape)
    (``lithe/quant.py:84-88``)."""
    from .kernels import search
    return search.encode(w, pools, proj)


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
