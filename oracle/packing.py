"""Oracle: 9-bit packed residency layout (test infrastructure only).

Restates ``lithe/kernels/packed.py:30-143`` and ``lithe/quant.py:23-43`` of the
reference. An adapter here is any object with ``modules`` (list of
``{"name", "shape_a", "shape_b"}``), ``indices`` (name -> {"A": (L, nA),
"B": (L, nB)} integer arrays), ``rank``, ``alpha``, ``num_levels`` and
``block_size`` attributes, or a dict with those keys.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Tuple

import numpy as np

INDEX_BITS = 9          # lithe/kernels/packed.py:30
PER_WORD = 7            # lithe/kernels/packed.py:31
INDEX_MASK = 0x1FF      # lithe/kernels/packed.py:32


def _get(ad, key, default=None):
    if isinstance(ad, dict):
        return ad.get(key, default)
    return getattr(ad, key, default)


def num_blocks(shape, block_size: int = 64) -> int:
    """ceil(prod(shape) / block_size), lithe/quant.py:39-43."""
    n = 1
    for s in shape:
        n *= int(s)
    return -(-n // block_size)


def blockify(w: np.ndarray, block_size: int = 64) -> np.ndarray:
    """Row-major flatten, zero-pad to a multiple of the block (lithe/quant.py:23-29)."""
    flat = np.asarray(w).reshape(-1)
    pad = (-flat.size) % block_size
    if pad:
        flat = np.concatenate([flat, np.zeros(pad, dtype=flat.dtype)])
    return flat.reshape(-1, block_size)


def unblockify(blocks: np.ndarray, shape) -> np.ndarray:
    """lithe/quant.py:32-36."""
    n = 1
    for s in shape:
        n *= int(s)
    return np.asarray(blocks).reshape(-1)[:n].reshape(tuple(int(s) for s in shape))


def pack(indices) -> np.ndarray:
    """Seven 9-bit fields per uint64, field j at bits [9j, 9j+9), last word zero-padded.

    lithe/kernels/packed.py:38-52. Raises ValueError for a value above 511.
    """
    flat = np.asarray(indices).reshape(-1).astype(np.uint64)
    if flat.size and int(flat.max()) > INDEX_MASK:
        raise ValueError("indices must be < 512 for 9-bit packing")
    n_words = -(-flat.size // PER_WORD)
    padded = np.zeros(n_words * PER_WORD, dtype=np.uint64)
    padded[:flat.size] = flat
    fields = padded.reshape(n_words, PER_WORD)
    words = np.zeros(n_words, dtype=np.uint64)
    for j in range(PER_WORD):
        words |= fields[:, j] << np.uint64(INDEX_BITS * j)
    return words


def unpack(words, n: int) -> np.ndarray:
    """Inverse of ``pack``: (n,) int64 (lithe/kernels/packed.py:55-60)."""
    w = np.asarray(words).astype(np.uint64).reshape(-1)
    shifts = (np.arange(PER_WORD, dtype=np.uint64) * np.uint64(INDEX_BITS))[None, :]
    fields = (w[:, None] >> shifts) & np.uint64(INDEX_MASK)
    return fields.reshape(-1)[:n].astype(np.int64)


@dataclass
class Layout:
    """Module offsets (in blocks) of one adapter's packed stream (lithe/kernels/packed.py:63-117)."""

    names: List[str]
    shapes_a: List[Tuple[int, int]]
    shapes_b: List[Tuple[int, int]]
    a_off: List[int]
    b_off: List[int]
    sides: np.ndarray          # (total_blocks,) int8: 0 = A block, 1 = B block
    num_levels: int
    block_size: int
    scaling: float

    @property
    def total_blocks(self) -> int:
        return int(self.sides.size)

    @property
    def num_indices(self) -> int:
        return self.total_blocks * self.num_levels

    @property
    def num_words(self) -> int:
        return -(-self.num_indices // PER_WORD)


def layout_of(ad) -> Layout:
    """Per module: A blocks then B blocks, modules in list order (lithe/kernels/packed.py:100-117)."""
    bs = int(_get(ad, "block_size", 64))
    names, sa, sb, a_off, b_off, sides = [], [], [], [], [], []
    cursor = 0
    for m in _get(ad, "modules"):
        na = num_blocks(m["shape_a"], bs)
        nb = num_blocks(m["shape_b"], bs)
        names.append(m["name"])
        sa.append(tuple(int(s) for s in m["shape_a"]))
        sb.append(tuple(int(s) for s in m["shape_b"]))
        a_off.append(cursor)
        b_off.append(cursor + na)
        sides.append(np.zeros(na, dtype=np.int8))
        sides.append(np.ones(nb, dtype=np.int8))
        cursor += na + nb
    sides_arr = np.concatenate(sides) if sides else np.zeros(0, dtype=np.int8)
    return Layout(names, sa, sb, a_off, b_off, sides_arr, int(_get(ad, "num_levels", 3)), bs,
                  float(_get(ad, "alpha")) / int(_get(ad, "rank")))


def stream_order(ad, layout: Layout) -> np.ndarray:
    """Indices in packed-stream order: (block, level)-major, A then B per module.

    lithe/kernels/packed.py:125-133.
    """
    idx = _get(ad, "indices")
    parts = []
    for name in layout.names:
        parts.append(np.asarray(idx[name]["A"]).T.reshape(-1))
        parts.append(np.asarray(idx[name]["B"]).T.reshape(-1))
    if not parts:
        return np.zeros(0, dtype=np.uint16)
    return np.concatenate(parts).astype(np.uint16)


def split_file_stream(stream, modules, num_levels: int, block_size: int = 64):
    """name -> {"A": (L, nA), "B": (L, nB)} from a ``.lithe`` index stream.

    lithe/fileio.py:136-150: the stream holds the A matrices of every module in header order,
    then the B matrices, each an (L, n_blocks) matrix in row-major order.
    """
    s = np.asarray(stream).reshape(-1)
    out = {m["name"]: {} for m in modules}
    cur = 0
    for side, key in (("A", "shape_a"), ("B", "shape_b")):
        for m in modules:
            c = num_levels * num_blocks(m[key], block_size)
            out[m["name"]][side] = s[cur:cur + c].reshape(num_levels, -1)
            cur += c
    if cur != s.size:
        raise ValueError(f"stream length {s.size} does not match the modules ({cur})")
    return out


def residency_from_file_stream(stream, modules, num_levels: int, block_size: int = 64) -> np.ndarray:
    """The ``.lithe`` stream reordered into the packed residency order (``split_file_stream``
    then ``stream_order``: lithe/fileio.py:136-150, lithe/kernels/packed.py:125-133)."""
    parts = split_file_stream(stream, modules, num_levels, block_size)
    ad = {"modules": modules, "indices": parts, "block_size": block_size, "num_levels": num_levels,
          "alpha": 1.0, "rank": 1}
    return stream_order(ad, layout_of(ad))


def pack_adapter(ad, layout: Layout = None):
    """(uint64 words, layout) for one adapter (lithe/kernels/packed.py:136-143)."""
    layout = layout or layout_of(ad)
    return pack(stream_order(ad, layout)), layout


def module_levels(words: np.ndarray, layout: Layout, name: str):
    """(idx_A (L, nA), idx_B (L, nB)) int64 of one module, read back from packed words."""
    i = layout.names.index(name)
    L = layout.num_levels
    flat = unpack(words, layout.num_indices).reshape(-1, L)
    na = num_blocks(layout.shapes_a[i], layout.block_size)
    nb = num_blocks(layout.shapes_b[i], layout.block_size)
    a = flat[layout.a_off[i]:layout.a_off[i] + na].T
    b = flat[layout.b_off[i]:layout.b_off[i] + nb].T
    return np.ascontiguousarray(a), np.ascontiguousarray(b)
