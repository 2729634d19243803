"""Dense factors from an adapter's index streams (``decode_factors`` of ``lithe/convert.py:15-29``).

The rest of the reference's conversion module (dense LoRA files, research
checkpoint import) is offline tooling outside this library.
"""
from __future__ import annotations

from typing import Dict, Tuple

import numpy as np
import torch

from . import codebook as cb
from . import quant
from .fileio import LitheAdapter


def adapter_pools(ad: LitheAdapter) -> Tuple[torch.Tensor, torch.Tensor]:
    return (cb.build_pools(ad.sigma_a, ad.block_size, ad.n_bits),
            cb.build_pools(ad.sigma_b, ad.block_size, ad.n_bits))


def decode_factors(ad: LitheAdapter, device="cuda") -> Dict[str, Tuple[torch.Tensor, torch.Tensor]]:
    """name -> (A_hat (r, d_in), B_hat (d_out, r)), float32, decoded on the GPU."""
    pool_a, pool_b = (p.to(device) for p in adapter_pools(ad))
    out = {}
    for m in ad.modules:
        idx = ad.indices[m["name"]]
        a = quant.decode(torch.from_numpy(idx["A"].astype(np.int32)).to(device), m["shape_a"], pool_a)
        b = quant.decode(torch.from_numpy(idx["B"].astype(np.int32)).to(device), m["shape_b"], pool_b)
        out[m["name"]] = (a, b)
    return out
