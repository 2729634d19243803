"""lithe_amd: MI355X-native index-resident multi-adapter LoRA (LITHE twin Hadamard codebook).

Drop-in for the reference's ``lithe`` inference path: same module names and
signatures (``lithe_amd.serve``, ``lithe_amd.module.LitheLinear``,
``lithe_amd.kernels``), computed by hand-written gfx950 HIP kernels behind the C
ABI of ``include/lithe_amd.h``.
"""
from .codebook import (BLOCK_SIZE, K, N_BITS, NUM_LEVELS, SIGMA_A, SIGMA_B, build_pools, codebook_sha256,
                       codewords, twin_pools)
from .fileio import LitheAdapter, load_lithe, read_header, save_lithe
from .kernels.packed import decode_factors
from .module import FLUX_TARGET_MODULES, LitheLinear, TwinCodebook, inject_lithe, lithe_layers

__version__ = "0.1.0"

__all__ = [
    "BLOCK_SIZE", "K", "N_BITS", "NUM_LEVELS", "SIGMA_A", "SIGMA_B",
    "build_pools", "codebook_sha256", "codewords", "twin_pools",
    "decode_factors",
    "LitheAdapter", "load_lithe", "read_header", "save_lithe",
    "FLUX_TARGET_MODULES", "LitheLinear", "TwinCodebook", "inject_lithe", "lithe_layers",
]
