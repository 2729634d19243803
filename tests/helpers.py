"""Shared test helpers: seeded random adapters (the reference's generator,
tests/test_kernels.py:20-28 of the reference) and comparison statistics."""
from __future__ import annotations

import numpy as np
import torch

from lithe_amd.fileio import LitheAdapter
from oracle import packing as opk

SMALL = [("blk.0.q", 128, 192), ("blk.0.mlp", 128, 320), ("blk.0.out", 320, 128), ("odd", 96, 40)]


def random_adapter(modules, rank, seed=0, levels=3):
    rng = np.random.default_rng(seed)
    mods, idx = [], {}
    for name, d_in, d_out in modules:
        sa, sb = [rank, d_in], [d_out, rank]
        mods.append({"name": name, "shape_a": sa, "shape_b": sb})
        idx[name] = {"A": rng.integers(0, 512, (levels, opk.num_blocks(sa))).astype(np.uint16),
                     "B": rng.integers(0, 512, (levels, opk.num_blocks(sb))).astype(np.uint16)}
    return LitheAdapter(modules=mods, indices=idx, rank=rank, alpha=float(rank), num_levels=levels)


def flux_modules(rank=16):
    """The 342 FLUX.1-dev target linears (19 double blocks x 12 + 38 single blocks x 3)."""
    mods = []
    for i in range(19):
        p = f"transformer_blocks.{i}."
        for n in ("attn.to_q", "attn.to_k", "attn.to_v", "attn.to_out.0",
                  "attn.add_q_proj", "attn.add_k_proj", "attn.add_v_proj", "attn.to_add_out"):
            mods.append((p + n, 3072, 3072))
        mods += [(p + "ff.net.0.proj", 3072, 12288), (p + "ff.net.2", 12288, 3072),
                 (p + "ff_context.net.0.proj", 3072, 12288), (p + "ff_context.net.2", 12288, 3072)]
    for i in range(38):
        p = f"single_transformer_blocks.{i}."
        mods += [(p + "attn.to_q", 3072, 3072), (p + "attn.to_k", 3072, 3072), (p + "attn.to_v", 3072, 3072)]
    return mods


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def rel(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def bf16_ulp(x) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (2^(e-7) for normal x)."""
    ax = np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(ax)) - 7)


def ulp_stats(got, want):
    """(max |diff| in bf16 ulps of want, fraction of elements that differ)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    d = np.abs(got - want)
    return float((d / bf16_ulp(want)).max()) if d.size else 0.0, float((d > 0).mean()) if d.size else 0.0
