"""Adapter index container and the ``.lithe`` file format (host side).

``LitheAdapter`` has the fields of ``lithe/fileio.py:34-58``. The file layout
is the reference's (``lithe/fileio.py:1-13``, ``README.md:206-212``)::

    b"LITHE001" | uint32 LE n | xz(UTF-8 JSON header), n bytes | xz(index stream)

The index stream is little-endian uint16: the A indices of every module in
header order, then the B indices, each module as its (L, n_blocks) matrix in
row-major order. The header carries the codebook parameters with the SHA-256
of the integer codeword table and the SHA-256 of the raw stream; loading
checks both.
"""
from __future__ import annotations

import hashlib
import json
import lzma
import struct
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Dict, List

import numpy as np

from . import codebook as cb

MAGIC = b"LITHE001"
LZMA_PRESET = 9 | lzma.PRESET_EXTREME


@dataclass
class LitheAdapter:
    """Index streams of one adapter plus everything needed to decode them."""

    modules: List[Dict[str, Any]]                 # [{"name", "shape_a", "shape_b"}] in stream order
    indices: Dict[str, Dict[str, np.ndarray]]      # name -> {"A": (L, nA), "B": (L, nB)} uint16
    rank: int
    alpha: float
    key_format: str = "diffusers"
    base_model: str = "black-forest-labs/FLUX.1-dev"
    block_size: int = cb.BLOCK_SIZE
    n_bits: int = cb.N_BITS
    num_levels: int = cb.NUM_LEVELS
    sigma_a: List[float] = field(default_factory=lambda: list(cb.SIGMA_A))
    sigma_b: List[float] = field(default_factory=lambda: list(cb.SIGMA_B))
    metadata: Dict[str, Any] = field(default_factory=dict)

    @property
    def num_indices(self) -> int:
        return sum(v["A"].size + v["B"].size for v in self.indices.values())

    def raw_stream(self) -> bytes:
        """All A matrices in module order, then all B matrices, as little-endian uint16."""
        names = [m["name"] for m in self.modules]
        chunks = [np.ascontiguousarray(self.indices[n][side], dtype="<u2").tobytes()
                  for side in ("A", "B") for n in names]
        return b"".join(chunks)


def _header(ad: LitheAdapter, raw: bytes) -> Dict[str, Any]:
    return {
        "format": "lithe",
        "version": 1,
        "codebook": {
            "name": "hadamard9-twin",
            "block_size": ad.block_size,
            "n_bits": ad.n_bits,
            "num_levels": ad.num_levels,
            "sigma_a": list(ad.sigma_a),
            "sigma_b": list(ad.sigma_b),
            "sha256": cb.codebook_sha256(ad.block_size, ad.n_bits),
        },
        "rank": ad.rank,
        "alpha": ad.alpha,
        "key_format": ad.key_format,
        "base_model": ad.base_model,
        "index_dtype": "uint16-le",
        "num_indices": ad.num_indices,
        "payload_sha256": hashlib.sha256(raw).hexdigest(),
        "modules": ad.modules,
        "metadata": ad.metadata,
    }


def save_lithe(path, ad: LitheAdapter) -> int:
    """Write ``ad`` to ``path``; returns the file size in bytes."""
    if ad.n_bits > 16:
        raise ValueError("uint16 streams need n_bits <= 16")
    raw = ad.raw_stream()
    head = lzma.compress(json.dumps(_header(ad, raw), separators=(",", ":")).encode("utf-8"),
                         preset=LZMA_PRESET)
    body = lzma.compress(raw, preset=LZMA_PRESET)
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "wb") as fh:
        fh.write(MAGIC + struct.pack("<I", len(head)) + head + body)
    return path.stat().st_size


def _read(path):
    with open(path, "rb") as fh:
        if fh.read(len(MAGIC)) != MAGIC:
            raise ValueError(f"{path}: not a .lithe file")
        (n,) = struct.unpack("<I", fh.read(4))
        header = json.loads(lzma.decompress(fh.read(n)).decode("utf-8"))
        return header, fh.read()


def read_header(path) -> Dict[str, Any]:
    return _read(path)[0]


def read_stream(path, verify: bool = True):
    """(header, index stream) of a ``.lithe`` file without splitting it per module.

    The stream is the file's little-endian uint16 index stream (A matrices of every module,
    then the B matrices), read-only. With ``verify`` the payload and codebook SHA-256 are
    checked as ``load_lithe`` does (``lithe/fileio.py:124-129``).
    """
    header, body = _read(path)
    raw = lzma.decompress(body)
    book = header["codebook"]
    if verify:
        if hashlib.sha256(raw).hexdigest() != header["payload_sha256"]:
            raise ValueError(f"{path}: payload checksum mismatch")
        if book["sha256"] != cb.codebook_sha256(book["block_size"], book["n_bits"]):
            raise ValueError(f"{path}: codebook hash mismatch")
    return header, np.frombuffer(raw, dtype="<u2")


def load_lithe(path, verify: bool = True) -> LitheAdapter:
    header, stream = read_stream(path, verify)
    book = header["codebook"]
    L, bs = int(book["num_levels"]), int(book["block_size"])
    modules = header["modules"]

    def count(shape):
        n = 1
        for s in shape:
            n *= int(s)
        return L * (-(-n // bs))

    counts_a = [count(m["shape_a"]) for m in modules]
    counts_b = [count(m["shape_b"]) for m in modules]
    if sum(counts_a) + sum(counts_b) != stream.size:
        raise ValueError(f"{path}: stream length {stream.size} does not match header")
    indices: Dict[str, Dict[str, np.ndarray]] = {m["name"]: {} for m in modules}
    cursor = 0
    for side, counts in (("A", counts_a), ("B", counts_b)):
        for m, c in zip(modules, counts):
            indices[m["name"]][side] = stream[cursor:cursor + c].reshape(L, -1).copy()
            cursor += c
    return LitheAdapter(modules=modules, indices=indices, rank=header["rank"], alpha=header["alpha"],
                        key_format=header["key_format"], base_model=header.get("base_model", ""),
                        block_size=bs, n_bits=book["n_bits"], num_levels=L, sigma_a=book["sigma_a"],
                        sigma_b=book["sigma_b"], metadata=header.get("metadata", {}))
