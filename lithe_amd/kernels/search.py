"""Nearest-codeword search and greedy residual encode on the GPU (API of ``lithe/kernels/search.py``).

All codewords of a level share one norm, so the nearest codeword of a block has bit q of its
index set exactly when the block's projection on the q-th Hadamard column is positive
(``lithe/quant.py:46-50``); the levels are searched greedily on the residual
(``lithe/quant.py:54-71``). One ``lithe_encode`` launch runs every level: a block is read once
and its indices (and, on request, its reconstruction) are written once.

The projection matrix must be the Hadamard generator of the codebook
(``lithe_amd.codebook.projection_matrix``): the kernel uses its closed form. Pools must be twin
Hadamard pools (any per-level scale), as for the decode.
"""
from __future__ import annotations

import ctypes
from typing import Tuple

import torch

from .. import codebook as cb
from .. import quant
from . import _hip

_PROJ = cb.projection_matrix()


def _check_proj(proj: torch.Tensor, block_size: int) -> None:
    if tuple(proj.shape) != tuple(_PROJ.shape) or block_size != _PROJ.shape[0]:
        raise ValueError(f"the GPU search needs the ({_PROJ.shape[0]}, {_PROJ.shape[1]}) Hadamard projection")
    if not torch.equal(proj.detach().to("cpu", torch.float32), _PROJ):
        raise ValueError("proj is not the codebook's Hadamard generator (lithe_amd.codebook.projection_matrix)")


def _encode(blocks: torch.Tensor, pools: torch.Tensor, want_recon: bool = True,
            idx_dtype: torch.dtype = torch.int64) -> Tuple[torch.Tensor, torch.Tensor]:
    _hip.require_gpu(blocks)
    if blocks.dim() != 2 or blocks.shape[1] != 64:
        raise ValueError("blocks must be (N, 64)")
    t = blocks.detach().to(torch.float32).contiguous()
    n = t.shape[0]
    lut = _hip.lut_from_pools(pools.to(t.device), torch.float32)
    idx = torch.empty((lut.num_levels, n), dtype=idx_dtype, device=t.device)
    recon = torch.empty((n, 64), dtype=torch.float32, device=t.device) if want_recon else None
    rc = _hip.load().lithe_encode(_hip.ptr(t), n, None, ctypes.byref(lut), None, _hip.ptr(idx),
                                  _hip.dtype_code(idx_dtype), n, 1, _hip.ptr(recon), _hip.stream_of(t.device))
    _hip.check(rc, "lithe_encode")
    return idx, recon


def lattice_search(blocks: torch.Tensor, proj: torch.Tensor, pool: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Nearest codeword of every block: (indices (N,) int64, codewords (N, B) fp32)
    (``lithe/kernels/search.py:65-83``). blocks (N, B); proj = U (B, n_bits); pool (K, B)."""
    n, bs = blocks.shape
    _check_proj(proj, bs)
    if pool.shape != (512, bs):
        raise ValueError("shape mismatch between blocks, proj and pool")
    idx, rec = _encode(blocks, pool.unsqueeze(0))
    return idx[0], rec


@torch.no_grad()
def rvq_encode_blocks_fast(blocks: torch.Tensor, pools: torch.Tensor,
                           proj: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Greedy twin RVQ: (indices (L, N) int64, reconstruction (N, B) fp32), all levels in one
    launch (``lithe/kernels/search.py:86-99``, ``lithe/quant.py:54-71``)."""
    _check_proj(proj, blocks.shape[1])
    return _encode(blocks, pools)


@torch.no_grad()
def encode(w: torch.Tensor, pools: torch.Tensor, proj: torch.Tensor = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Row-major blockify (zero-padded), encode, and the decoded reconstruction in ``w``'s shape:
    (indices (L, n_blocks) int64, w_hat) (``lithe/quant.py:84-88``)."""
    if proj is not None:
        _check_proj(proj, pools.shape[-1])
    idx, rec = _encode(quant.blockify(w.to(torch.float32)), pools)
    return idx, quant.unblockify(rec, w.shape)
