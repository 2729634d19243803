"""The reference's multi-adapter serving forward restated with torch CPU ops.

TEST INFRASTRUCTURE ONLY: the CPU baseline of ``bench.py`` (its ``cpu_baseline`` leg) and a
cross-check in ``tests/``; the product never imports it.

``lithe/serve.py:63-97`` (``MultiAdapterLinear.forward``) on the CPU: the adapters active in
the batch are decoded from their level-major integer index tensors by an fp32 gather-sum over
the levels in level order (``lithe/quant.py:74-81, 91-92``); B is multiplied by the adapter's
alpha / r in fp32 and both factors by the square root of the route weight; the factors of every
sample are stacked along the rank and cast to the activation dtype; then ``x A^T`` and its
product with ``B^T`` run as two ``torch.bmm`` in the activation dtype and the delta is added to
the base output. The numbers equal ``oracle.delta.serve_forward`` up to the accumulation order
of the matrix products (checked in ``tests/test_oracle.py``).
"""
from __future__ import annotations

from typing import Sequence, Tuple

import torch


def decode_factor(idx: torch.Tensor, pools: torch.Tensor, shape: Tuple[int, int]) -> torch.Tensor:
    """(L, n_blocks) integer indices -> fp32 factor of ``shape``: pools[0][i0] + pools[1][i1] + ...
    summed in level order, then the blocks laid out row-major (``lithe/quant.py:23-43, 74-81``)."""
    lev = idx.long()
    acc = pools[0].index_select(0, lev[0])
    for level in range(1, lev.shape[0]):
        acc = acc + pools[level].index_select(0, lev[level])
    n = shape[0] * shape[1]
    return acc.reshape(-1)[:n].reshape(shape)


def routed_add(x: torch.Tensor, out: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
               idx_a: Sequence[torch.Tensor], idx_b: Sequence[torch.Tensor], scales: torch.Tensor,
               pool_a: torch.Tensor, pool_b: torch.Tensor, rank: int) -> torch.Tensor:
    """``out + delta`` of a routed batch.

    x (b, M, d_in) and out (b, M, d_out) in the activation dtype; ids (b, m) adapter ids
    (-1 = empty entry) and weights (b, m) fp32; idx_a[j] / idx_b[j] the (L, n_blocks) indices of
    adapter j; scales[j] its alpha / r; pools (L, K, block) fp32.
    """
    valid = ids >= 0
    if not bool(valid.any()):
        return out.clone()
    bsz, m = ids.shape
    d_in, d_out = x.shape[-1], out.shape[-1]
    active = torch.unique(ids[valid]).tolist()
    a_dec = {j: decode_factor(idx_a[j], pool_a, (rank, d_in)) for j in active}
    b_dec = {j: decode_factor(idx_b[j], pool_b, (d_out, rank)) * scales[j] for j in active}
    g = (weights * valid).clamp(min=0).sqrt()
    zero_a = torch.zeros(rank, d_in)
    zero_b = torch.zeros(d_out, rank)
    a_rows, b_cols = [], []
    for i in range(bsz):
        ar, bc = [], []
        for k in range(m):
            j = int(ids[i, k])
            ar.append(a_dec[j] * g[i, k] if j >= 0 else zero_a)
            bc.append(b_dec[j] * g[i, k] if j >= 0 else zero_b)
        a_rows.append(torch.cat(ar, 0))
        b_cols.append(torch.cat(bc, 1))
    a_s = torch.stack(a_rows).to(x.dtype)                   # (b, m r, d_in)
    b_s = torch.stack(b_cols).to(x.dtype)                   # (b, d_out, m r)
    xs = x.reshape(bsz, -1, d_in)
    mid = torch.bmm(xs, a_s.transpose(1, 2).contiguous())
    delta = torch.bmm(mid, b_s.transpose(1, 2).contiguous())
    return out + delta.reshape(out.shape)
