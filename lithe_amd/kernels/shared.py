"""Index-resident per-sample LoRA delta, decode fused into the shrink / expand tiles.

API of ``lithe/kernels/shared.py``. Each wrapped linear keeps, for every
resident adapter, only index tensors ``idx_A`` (n_slots, L, n_blocks_A) and
``idx_B`` (n_slots, L, n_blocks_B) plus one pair of codebook pools; sample b
uses adapter ``assign[b]``::

    A_j[r, d] = sum_l pool_A[l, idx_A[j, l, blk(r, d)], pos(r, d)]
    delta[b]  = scaling * (x_b @ A_j.T) @ B_j.T

The gfx950 kernels (``lithe_lora_delta``) never store A or B: the shrink
decodes one 16-value period per (rank, block) into LDS, the expand decodes its
B tile into LDS, both from the closed form of the codewords. Dtype steps are
the reference's (``shared.py:177-194``): pools cast to the activation dtype,
factor = fp32 level sum cast to the activation dtype, y_lo rounded to the
activation dtype, delta rounded to ``out_dtype``, then ``* scaling``.

``packed_lora_delta`` is the same delta read straight from a bit-packed bank
(the residency form of ``lithe/kernels/packed.py``), the north-star path.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _delta, _hip


def _check(x, idx_A, pools_A, idx_B, pools_B, assign, R, D_out):
    """Shape validation with the reference's messages (shared.py:160-174)."""
    if x.dim() != 3:
        raise ValueError(f"x must be (B, M, D_in), got {tuple(x.shape)}")
    bsz, _, d_in = x.shape
    L, _, bs = pools_A.shape
    if pools_B.shape != pools_A.shape:
        raise ValueError("pools_A and pools_B must have the same (L, K, B) shape")
    if idx_A.dim() != 3 or idx_B.dim() != 3 or idx_A.shape[1] != L or idx_B.shape[1] != L:
        raise ValueError("index pools must be (n_slots, L, n_blocks)")
    if R * d_in != idx_A.shape[2] * bs or D_out * R != idx_B.shape[2] * bs:
        raise ValueError("index pools do not match (R, D_in, D_out)")
    if d_in % bs or (D_out * R) % bs:
        raise ValueError("d_in and d_out * r must be multiples of the block size")
    if assign.shape != (bsz,):
        raise ValueError(f"assign must be ({bsz},)")


def _act_dtype(x: torch.Tensor) -> None:
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"lithe_amd kernels take bfloat16 or float32 activations, got {x.dtype}")


def _slots(assign: torch.Tensor, device) -> torch.Tensor:
    a = assign.to(device=device, dtype=torch.int32)
    return a.reshape(-1, 1).contiguous()


def _level_idx(idx: torch.Tensor) -> torch.Tensor:
    if idx.dtype in (torch.int32, torch.int16) and idx.stride(-1) == 1:
        return idx
    return idx.to(torch.int32).contiguous()


def shared_codebook_lora_delta(x: torch.Tensor, idx_A: torch.Tensor, pools_A: torch.Tensor,
                               idx_B: torch.Tensor, pools_B: torch.Tensor, assign: torch.Tensor,
                               R: int, D_out: int, scaling: float,
                               out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Per-sample LoRA delta ``(B, M, D_out)`` decoded on the fly from index pools (GPU only).

    x (B, M, D_in); idx_A (n_slots, L, n_blocks_A) and idx_B (n_slots, L, n_blocks_B)
    integer; pools (L, K, block) float; assign (B,) adapter slot per sample.
    """
    _check(x, idx_A, pools_A, idx_B, pools_B, assign, R, D_out)
    _hip.require_gpu(x, idx_A, idx_B, assign)
    _act_dtype(x)
    out_dtype = out_dtype or x.dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"out_dtype must be bfloat16 or float32, got {out_dtype}")
    L = int(pools_A.shape[0])
    ia, ib = _level_idx(idx_A), _level_idx(idx_B)
    x_c = x.contiguous()
    f = _delta.indexed_factors(_delta.index_source(ia, L, ia.shape[2]), _delta.index_source(ib, L, ib.shape[2]),
                               _hip.lut_from_pools(pools_A, x.dtype), _hip.lut_from_pools(pools_B, x.dtype))
    slots = _slots(assign, x.device)
    out = torch.empty((x.shape[0], x.shape[1], D_out), dtype=out_dtype, device=x.device)
    return _delta.lora_delta(x_c, out, rank=R, factors=f, route=_delta.routes(slots), accumulate=False,
                             out_scale=float(scaling))


def packed_lora_delta(x: torch.Tensor, bank: torch.Tensor, a_off: int, b_off: int, num_levels: int,
                      pools: Tuple[torch.Tensor, torch.Tensor], assign: torch.Tensor, R: int, D_out: int,
                      scaling: float, out: Optional[torch.Tensor] = None, accumulate: bool = False,
                      out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Per-sample LoRA delta decoded from a packed bank (n_slots, n_words) uint64.

    ``a_off`` / ``b_off`` are the module's block offsets in the layout. With
    ``accumulate`` the delta is added into ``out`` (the base output) with the
    rounding of ``out + delta`` (lithe/kernels/layers.py:131); otherwise the delta
    is returned (written into ``out`` when given).
    """
    if x.dim() != 3:
        raise ValueError(f"x must be (B, M, D_in), got {tuple(x.shape)}")
    _hip.require_gpu(x, bank, assign)
    _act_dtype(x)
    if assign.shape != (x.shape[0],):
        raise ValueError(f"assign must be ({x.shape[0]},)")
    if x.shape[2] % 64 or (D_out * R) % 64:
        raise ValueError("d_in and d_out * r must be multiples of the block size")
    pa, pb = pools
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs the base output in `out`")
        out = torch.empty((x.shape[0], x.shape[1], D_out), dtype=out_dtype or x.dtype, device=x.device)
    elif out.shape != (x.shape[0], x.shape[1], D_out) or not out.is_contiguous():
        raise ValueError("out must be a contiguous (B, M, D_out) tensor")
    f = _delta.indexed_factors(_delta.packed_source(bank, num_levels, a_off),
                               _delta.packed_source(bank, num_levels, b_off),
                               _hip.lut_from_pools(pa, x.dtype), _hip.lut_from_pools(pb, x.dtype))
    return _delta.lora_delta(x.contiguous(), out, rank=R, factors=f, route=_delta.routes(_slots(assign, x.device)),
                             accumulate=accumulate, out_scale=float(scaling))
