"""Oracle: per-sample LoRA deltas with the reference's dtype steps (test infrastructure only).

Every function follows the rounding sequence of the reference function it
cites: where the reference rounds an intermediate to the activation dtype, the
oracle rounds there too. Matrix products are evaluated in float64 and then
rounded the way the reference rounds its fp32-accumulated product; the
reference's own accumulation order is unspecified (Triton / cuBLAS), so tests
compare the GPU results with a stated tolerance, not bit for bit.

Dtypes are named by strings: "bf16" or "fp32". Activations are passed as fp32
arrays whose values are already representable in that dtype.
"""
from __future__ import annotations

import numpy as np

from . import packing
from .decode import round_to, rvq_decode


def _decode_factor(levels, pools, shape) -> np.ndarray:
    """fp32 factor from level-major indices (L, n_blocks), sum in level order."""
    return packing.unblockify(rvq_decode(levels, pools), shape)


def shared_delta(x, idx_A, pools_A, idx_B, pools_B, assign, R, D_out, scaling,
                 x_dtype="bf16", out_dtype=None) -> np.ndarray:
    """lithe/kernels/shared.py:177-194 (``shared_codebook_lora_delta_reference``).

    Steps: pools cast to the activation dtype; factor = fp32 level sum of the
    cast pools, cast to the activation dtype; y_lo = x A^T rounded to the
    activation dtype; delta = y_lo B^T rounded to ``out_dtype``; then
    ``delta * scaling`` in ``out_dtype`` when scaling != 1.
    """
    out_dtype = out_dtype or x_dtype
    x = np.asarray(x, dtype=np.float32)
    bsz, _, d_in = x.shape
    pa = round_to(np.asarray(pools_A, dtype=np.float32), x_dtype)
    pb = round_to(np.asarray(pools_B, dtype=np.float32), x_dtype)
    out = []
    for b in range(bsz):
        j = int(assign[b])
        a = round_to(_decode_factor(np.asarray(idx_A[j]), pa, (R, d_in)), x_dtype)
        bm = round_to(_decode_factor(np.asarray(idx_B[j]), pb, (D_out, R)), x_dtype)
        y = round_to(x[b].astype(np.float64) @ a.astype(np.float64).T, x_dtype)
        out.append(round_to(y.astype(np.float64) @ bm.astype(np.float64).T, out_dtype))
    delta = np.stack(out)
    if scaling != 1.0:
        delta = round_to(delta * np.float32(scaling), out_dtype)
    return delta


def index_linear(base_out, delta, x_dtype="bf16") -> np.ndarray:
    """lithe/kernels/layers.py:131: ``out + delta`` in the activation dtype."""
    return round_to(np.asarray(base_out, dtype=np.float32) + delta, x_dtype)


def serve_forward(x, base_out, ids, weights, idx_a, idx_b, scales, pool_a, pool_b, rank,
                  x_dtype="fp32") -> np.ndarray:
    """lithe/serve.py:69-97 (``MultiAdapterLinear.forward``), rank-stacked mixture routing.

    ids (b, m) with -1 = padding, weights (b, m); idx_a (n, L, nA), idx_b (n, L, nB)
    level-major; scales (n,) = alpha / r. Factors are decoded with fp32 pools;
    B is multiplied by its scale in fp32; both factors by sqrt(w) in fp32; the
    stacked factors are cast to the activation dtype; x A^T is rounded to the
    activation dtype, then (x A^T) B^T, then out + delta.
    """
    x = np.asarray(x, dtype=np.float32)
    ids = np.asarray(ids)
    w = np.asarray(weights, dtype=np.float32)
    out = np.asarray(base_out, dtype=np.float32)
    if (ids < 0).all():
        return out.copy()
    bsz = ids.shape[0]
    d_in = x.shape[-1]
    xs = x.reshape(bsz, -1, d_in)
    out3 = out.reshape(bsz, xs.shape[1], -1)
    d_out = out3.shape[-1]
    pa = np.asarray(pool_a, dtype=np.float32)
    pb = np.asarray(pool_b, dtype=np.float32)
    res = np.empty_like(out3)
    for i in range(bsz):
        a_rows, b_cols = [], []
        for j in range(ids.shape[1]):
            if ids[i, j] < 0:
                continue
            g = np.sqrt(np.maximum(w[i, j], np.float32(0)))           # fp32 sqrt
            a = _decode_factor(np.asarray(idx_a[ids[i, j]]), pa, (rank, d_in))
            bm = _decode_factor(np.asarray(idx_b[ids[i, j]]), pb, (d_out, rank))
            bm = bm * np.float32(scales[ids[i, j]])
            a_rows.append(round_to(a * g, x_dtype))
            b_cols.append(round_to(bm * g, x_dtype))
        if not a_rows:
            res[i] = out3[i]
            continue
        a_s = np.concatenate(a_rows, axis=0).astype(np.float64)       # (m r, d_in)
        b_s = np.concatenate(b_cols, axis=1).astype(np.float64)       # (d_out, m r)
        mid = round_to(xs[i].astype(np.float64) @ a_s.T, x_dtype)
        delta = round_to(mid.astype(np.float64) @ b_s.T, x_dtype)
        res[i] = round_to(out3[i] + delta, x_dtype)
    return res.reshape(out.shape)


def per_sample_delta(x, sA, sB, scaling, x_dtype="bf16") -> np.ndarray:
    """lithe/kernels/sgmv.py:103-160 (``per_sample_lora_delta``).

    bf16 (the kernel path, sgmv.py:29-100): mid = bf16(fp32(x A^T) * scale_b)
    with the scale read as bf16; delta = bf16(mid B^T).
    fp32 (the bmm path, sgmv.py:103-109): mid = x A^T; delta = (mid B^T) * scale_b.
    """
    x = np.asarray(x, dtype=np.float32)
    a = round_to(np.asarray(sA, dtype=np.float32), x_dtype).astype(np.float64)
    bm = round_to(np.asarray(sB, dtype=np.float32), x_dtype).astype(np.float64)
    s = round_to(np.asarray(scaling, dtype=np.float32), x_dtype)
    out = []
    for b in range(x.shape[0]):
        acc = x[b].astype(np.float64) @ a[b].T
        if x_dtype == "bf16":
            mid = round_to(np.float32(acc) * s[b], "bf16")
            out.append(round_to(mid.astype(np.float64) @ bm[b].T, "bf16"))
        else:
            mid = np.float32(acc)
            d = np.float32(mid.astype(np.float64) @ bm[b].T)
            out.append(d * s[b])
    return np.stack(out)


def lithe_linear(x, base_out, a_hat, b_hat, scaling, x_dtype="bf16") -> np.ndarray:
    """lithe/module.py:145-156 (inference): base + (x A^T) B^T * scaling.

    F.linear rounds each product to the activation dtype; ``delta * scaling``
    and the final add round again.
    """
    x = np.asarray(x, dtype=np.float32)
    a = round_to(np.asarray(a_hat, dtype=np.float32), x_dtype).astype(np.float64)
    bm = round_to(np.asarray(b_hat, dtype=np.float32), x_dtype).astype(np.float64)
    mid = round_to(x.astype(np.float64) @ a.T, x_dtype)
    delta = round_to(mid.astype(np.float64) @ bm.T, x_dtype)
    delta = round_to(delta * np.float32(scaling), x_dtype)
    return round_to(np.asarray(base_out, dtype=np.float32) + delta, x_dtype)


def truth_delta(x, a, b) -> np.ndarray:
    """float64 closed form x A^T B^T of one sample (no intermediate rounding)."""
    return np.asarray(x, np.float64) @ np.asarray(a, np.float64).T @ np.asarray(b, np.float64).T
