"""Oracle: residual decode and the bf16 cast (test infrastructure only).

Restates ``lithe/quant.py:74-92`` and ``lithe/kernels/packed.py:241-269`` of the
reference. The fp32 sum runs in level order, ``(p0 + p1) + p2``
(``lithe/quant.py:78-80``, ``lithe/kernels/packed.py:248-249``); numpy float32
addition is IEEE round-to-nearest-even with no contraction, as torch's is.
"""
from __future__ import annotations

import numpy as np

from . import packing


# ----------------------------------------------------------------------------- bf16
def bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even; NaN stays NaN.

    This is the rounding of torch's ``Tensor.to(torch.bfloat16)``.
    """
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        r = np.where(nan, ((u >> np.uint64(16)) | np.uint64(0x40)).astype(np.uint16), r)
    return r


def bf16_value(bits) -> np.ndarray:
    """bf16 bit patterns -> fp32 values (exact)."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)


def round_bf16(x) -> np.ndarray:
    """fp32 values rounded to bf16 and widened back to fp32."""
    return bf16_value(bf16_bits(x))


def round_to(x, dtype: str) -> np.ndarray:
    """Round fp32 values to the activation dtype ("bf16" or "fp32")."""
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "fp32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(dtype)


# ----------------------------------------------------------------------------- decode
def rvq_decode(indices, pools) -> np.ndarray:
    """indices (L, N) -> (N, block) fp32: pools[0][i0] + pools[1][i1] + ... in order.

    lithe/quant.py:74-81.
    """
    idx = np.asarray(indices).astype(np.int64)
    p = np.asarray(pools, dtype=np.float32)
    out = p[0][idx[0]].copy()
    for level in range(1, idx.shape[0]):
        out += p[level][idx[level]]
    return out


def decode(indices, shape, pools) -> np.ndarray:
    """lithe/quant.py:91-92: decode then unblockify to ``shape``."""
    return packing.unblockify(rvq_decode(indices, pools), shape)


def decode_flat(flat, layout: packing.Layout, pool_a, pool_b) -> np.ndarray:
    """fp32 (total_blocks, block) from a flat (block, level)-major index stream.

    lithe/kernels/packed.py:241-250: the side of every block picks pool A or B,
    and the levels are summed in order.
    """
    L = layout.num_levels
    idx = np.asarray(flat).astype(np.int64).reshape(layout.total_blocks, L)
    is_b = layout.sides.astype(bool)[:, None]
    pa = np.asarray(pool_a, dtype=np.float32)
    pb = np.asarray(pool_b, dtype=np.float32)
    out = np.zeros((layout.total_blocks, pa.shape[-1]), dtype=np.float32)
    for level in range(L):
        out += np.where(is_b, pb[level][idx[:, level]], pa[level][idx[:, level]])
    return out


def decode_packed(words, layout: packing.Layout, pool_a, pool_b) -> np.ndarray:
    """fp32 decode of one packed adapter (lithe/kernels/packed.py:253-257)."""
    return decode_flat(packing.unpack(words, layout.num_indices), layout, pool_a, pool_b)


def split_decoded(out, layout: packing.Layout):
    """name -> (A (r, d_in), B (d_out, r)) views (lithe/kernels/packed.py:260-269)."""
    flat = np.asarray(out).reshape(-1)
    bs = layout.block_size
    res = {}
    for name, sa, sb, ao, bo in zip(layout.names, layout.shapes_a, layout.shapes_b,
                                    layout.a_off, layout.b_off):
        na, nb = sa[0] * sa[1], sb[0] * sb[1]
        res[name] = (flat[ao * bs:ao * bs + na].reshape(sa), flat[bo * bs:bo * bs + nb].reshape(sb))
    return res
