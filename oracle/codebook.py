"""Oracle: the deterministic twin Hadamard codebook (test infrastructure only).

Restates ``lithe/codebook.py:27-94`` and the specification at
``README.md:192-200`` of the reference:

    H_syl            order-64 Sylvester-Hadamard matrix
    U = H_syl[:, :9] 64 x 9 generator
    s_k[q] = +1 if bit q of k is set, else -1        (k in [0, 512))
    3 c_k  = U s_k                                     (exact integers, int8)
    pool_side[l] = fp32( sigma_side[l] * (3 c_k / 3.0) ) computed in float64

The Hadamard matrix is built here by the doubling recursion
H_{2n} = [[H, H], [H, -H]], not by the popcount parity the reference uses, so
the two constructions check each other (and both equal
``scipy.linalg.hadamard``).
"""
from __future__ import annotations

import hashlib

import numpy as np

BLOCK_SIZE = 64
N_BITS = 9
K = 1 << N_BITS
NUM_LEVELS = 3
SIGMA_A = (0.06, 0.06, 0.06)            # lithe/codebook.py:31
SIGMA_B = (0.0025, 0.001, 0.0005)       # lithe/codebook.py:32

# SHA-256 of the int8 (512, 64) table 3c_k, pinned by the reference's own test
# (tests/test_codebook.py:9).
INT_TABLE_SHA256 = "eb1f4de0d64df9980436232299238e56ff04efa9ab075ded3f72c2a821ad0301"


def hadamard(n: int = BLOCK_SIZE) -> np.ndarray:
    """Sylvester-Hadamard matrix of order ``n`` by doubling (lithe/codebook.py:35-42)."""
    if n <= 0 or n & (n - 1):
        raise ValueError(f"n must be a power of two, got {n}")
    h = np.ones((1, 1), dtype=np.int64)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h.astype(np.int8)


def generator(block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> np.ndarray:
    """U = first ``n_bits`` columns of H_syl (lithe/codebook.py:45-49)."""
    return np.ascontiguousarray(hadamard(block_size)[:, :n_bits])


def signs(n_bits: int = N_BITS) -> np.ndarray:
    """s_k for all k, (2**n_bits, n_bits) int8, +1 where bit q is set (lithe/codebook.py:52-56)."""
    k = np.arange(1 << n_bits)
    out = np.empty((1 << n_bits, n_bits), dtype=np.int8)
    for q in range(n_bits):
        out[:, q] = np.where((k >> q) & 1, 1, -1)
    return out


def integer_table(block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> np.ndarray:
    """3 c_k = U s_k as int8 (K, block_size) (lithe/codebook.py:59-63)."""
    u = generator(block_size, n_bits).astype(np.int64)
    s = signs(n_bits).astype(np.int64)
    return (s @ u.T).astype(np.int8)


def table_sha256(block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> str:
    """lithe/codebook.py:92-94."""
    return hashlib.sha256(integer_table(block_size, n_bits).tobytes()).hexdigest()


def pools(scales, block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> np.ndarray:
    """fp32 (L, K, block_size) pools: float64 (int / 3.0) times sigma, then one cast.

    The operation order (divide by sqrt(9) = 3.0 first, multiply by the scale in
    float64, a single cast to fp32) is the reference's (lithe/codebook.py:72-77).
    """
    c = integer_table(block_size, n_bits).astype(np.float64) / np.sqrt(n_bits)
    return np.stack([float(s) * c for s in scales]).astype(np.float32)


def twin_pools(sigma_a=SIGMA_A, sigma_b=SIGMA_B):
    """(pool_A, pool_B), lithe/codebook.py:80-84."""
    return pools(sigma_a), pools(sigma_b)
