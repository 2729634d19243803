"""Oracle: nearest-codeword search and greedy residual encode (test infrastructure only).

Restates ``lithe/quant.py:46-71`` (``nearest_index``, ``rvq_encode_blocks``) and
``lithe/kernels/search.py:58-62`` (``lattice_search_reference``). The projections are formed in
float64 from the fp32 residual (the reference forms them in fp32 with a BLAS-defined order, so
the two can disagree only where a projection is within fp32 rounding of zero; ``margin``
reports the smallest |projection| so that tests can set such blocks apart). The residual and
the reconstruction are updated in fp32 in level order, as the reference does.

Pinned by a brute-force nearest-codeword search over all 512 codewords (``cdist_nearest``),
exact round trips of lattice points, and the per-coordinate error recursion of the nine
orthogonal Hadamard directions (``tests/test_search.py``).
"""
from __future__ import annotations

import numpy as np

from . import codebook


def projection_matrix() -> np.ndarray:
    """U (64, 9) +-1: the first nine Sylvester-Hadamard columns (lithe/codebook.py:45-49, 87-89)."""
    return codebook.hadamard(64)[:, :9].astype(np.float64)


def nearest_index(x, proj=None):
    """(indices (N,) int64, projections (N, 9) float64) of the closed-form search (lithe/quant.py:46-50)."""
    u = projection_matrix() if proj is None else np.asarray(proj, np.float64)
    ip = np.asarray(x, np.float64) @ u
    idx = ((ip > 0).astype(np.int64) << np.arange(u.shape[1], dtype=np.int64)).sum(axis=1)
    return idx, ip


def rvq_encode_blocks(blocks, pools):
    """(indices (L, N) int64, reconstruction (N, 64) fp32, margin (N,)) of the greedy encode
    (lithe/quant.py:54-71); margin = smallest |projection| over all levels of a block."""
    residual = np.asarray(blocks, np.float32).copy()
    p = np.asarray(pools, np.float32)
    recon = np.zeros_like(residual)
    out, margin = [], np.full(residual.shape[0], np.inf)
    for level in range(p.shape[0]):
        idx, ip = nearest_index(residual)
        margin = np.minimum(margin, np.abs(ip).min(axis=1))
        sel = p[level][idx]
        recon += sel
        residual = residual - sel
        out.append(idx)
    return np.stack(out), recon, margin


def cdist_nearest(x, pool) -> np.ndarray:
    """Brute force: index of the codeword of ``pool`` (512, 64) closest to each row of x."""
    x = np.asarray(x, np.float64)
    c = np.asarray(pool, np.float64)
    d = (x * x).sum(1)[:, None] - 2.0 * x @ c.T + (c * c).sum(1)[None, :]
    return d.argmin(axis=1)
