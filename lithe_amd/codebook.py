"""The deterministic Hadamard 9-bit twin codebook (host-side constants).

Same definition and API as ``lithe/codebook.py:1-94`` of the reference: for an
index k in [0, 512) and a coordinate t in [0, 64),

    3 c_k[t] = sum_{q<9} H_syl[t, q] s_k[q],   H_syl[t, q] = (-1)^popcount(t & q),
    s_k[q]   = +1 if bit q of k is set, else -1.

This module evaluates it in the closed form the GPU kernels use: with m_t the
9-bit mask whose bit q is [popcount(t & q) is even], a term is +1 exactly where
bit q of k equals bit q of m_t, so 3 c_k[t] = 9 - 2 popcount((k ^ m_t) & 511).
Pools are fp32(sigma_l * (3 c / 3.0)) computed in float64, the reference's
operation order, so they are bit-identical to the reference's pools.
"""
from __future__ import annotations

import hashlib
from typing import Sequence, Tuple

import numpy as np
import torch

BLOCK_SIZE = 64
N_BITS = 9
K = 1 << N_BITS
NUM_LEVELS = 3
SIGMA_A: Tuple[float, ...] = (0.06, 0.06, 0.06)
SIGMA_B: Tuple[float, ...] = (0.0025, 0.001, 0.0005)


def _parity(v: np.ndarray) -> np.ndarray:
    return (np.bitwise_count(v) & 1).astype(np.int64)


def sylvester_hadamard(n: int) -> np.ndarray:
    """H[t, j] = (-1)^popcount(t & j), the order-n Sylvester-Hadamard matrix (int8)."""
    if n <= 0 or n & (n - 1):
        raise ValueError(f"n must be a power of two, got {n}")
    t = np.arange(n, dtype=np.uint64)
    return (1 - 2 * _parity(t[:, None] & t[None, :])).astype(np.int8)


def hadamard_generator(block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> np.ndarray:
    """U = first ``n_bits`` columns of H_syl, (block_size, n_bits) int8."""
    if block_size < n_bits:
        raise ValueError("block_size must be >= n_bits")
    return np.ascontiguousarray(sylvester_hadamard(block_size)[:, :n_bits])


def sign_table(n_bits: int = N_BITS) -> np.ndarray:
    """s_k for every k, (2**n_bits, n_bits) int8, +1 where bit q of k is set."""
    k = np.arange(1 << n_bits)[:, None]
    q = np.arange(n_bits)[None, :]
    return (2 * ((k >> q) & 1) - 1).astype(np.int8)


def sign_masks(block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> np.ndarray:
    """m_t for every coordinate t: bit q set iff popcount(t & q) is even; (block_size,) uint32."""
    t = np.arange(block_size, dtype=np.uint32)[:, None]
    q = np.arange(n_bits, dtype=np.uint32)[None, :]
    even = (1 - _parity(t & q)).astype(np.uint32)
    return (even << q).sum(axis=1).astype(np.uint32)


def mismatch_counts(block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> np.ndarray:
    """popcount((k ^ m_t) & (2**n_bits - 1)) for every (k, t); (K, block_size) int64."""
    k = np.arange(1 << n_bits, dtype=np.uint32)[:, None]
    m = sign_masks(block_size, n_bits)[None, :]
    return np.bitwise_count((k ^ m) & np.uint32((1 << n_bits) - 1)).astype(np.int64)


def integer_codewords(block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> np.ndarray:
    """sqrt(n_bits) * c_k = n_bits - 2 * mismatch count, exact integers, (K, block_size) int8."""
    return (n_bits - 2 * mismatch_counts(block_size, n_bits)).astype(np.int8)


def codewords(block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> torch.Tensor:
    """Unit-variance codeword matrix C, (K, block_size) float32."""
    c = integer_codewords(block_size, n_bits).astype(np.float64) / np.sqrt(n_bits)
    return torch.from_numpy(c.astype(np.float32))


def build_pools(scales: Sequence[float], block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> torch.Tensor:
    """Stack of scaled pools, (len(scales), K, block_size) float32."""
    c = integer_codewords(block_size, n_bits).astype(np.float64) / np.sqrt(n_bits)
    return torch.from_numpy(np.stack([float(s) * c for s in scales]).astype(np.float32))


def twin_pools(block_size: int = BLOCK_SIZE, n_bits: int = N_BITS, sigma_a: Sequence[float] = SIGMA_A,
               sigma_b: Sequence[float] = SIGMA_B) -> Tuple[torch.Tensor, torch.Tensor]:
    """(pool_A, pool_B), each (L, K, block_size) float32."""
    return build_pools(sigma_a, block_size, n_bits), build_pools(sigma_b, block_size, n_bits)


def projection_matrix(block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> torch.Tensor:
    """U as float32 (block_size, n_bits)."""
    return torch.from_numpy(hadamard_generator(block_size, n_bits).astype(np.float32))


def codebook_sha256(block_size: int = BLOCK_SIZE, n_bits: int = N_BITS) -> str:
    """SHA-256 of the exact integer codeword table (int8, row-major)."""
    return hashlib.sha256(integer_codewords(block_size, n_bits).tobytes()).hexdigest()


def value_table(scales: Sequence[float], n_bits: int = N_BITS) -> np.ndarray:
    """(L, n_bits + 1) fp32: the pool value of a coordinate with mismatch count p, per level."""
    p = np.arange(n_bits + 1, dtype=np.float64)
    c = (n_bits - 2 * p) / np.sqrt(n_bits)
    return np.stack([float(s) * c for s in scales]).astype(np.float32)
