"""Bit-packed GPU residency and the bulk decode (API of ``lithe/kernels/packed.py``).

Residency form (reference ``lithe/kernels/packed.py:1-9``): the index stream of
one adapter is (block, level)-major; each index is 9 bits and 7 share one
uint64 word, index p at bits [9(p % 7), 9(p % 7) + 9) of word p // 7, bit 63
always 0. Adapters covering the same modules with the same shapes share one
``PackedLayout``. The 342-linear FLUX.1-dev layout at rank 16 holds 2,101,248
indices = 300,179 words = 2.40 MB per adapter.

Decode (``lithe_decode``, gfx950): each thread decodes the 8 distinct values
of half a 64-value block (codewords have period 16) and stores them to their 4
positions; fp32 level sum in order, one round-to-nearest-even cast to bf16, so
the output equals ``quant.decode(...).to(bfloat16)`` bit for bit.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from .. import quant
from . import _hip

INDEX_BITS = 9
PER_WORD = 7          # 7 x 9 = 63 bits per uint64 word
INDEX_MASK = (1 << INDEX_BITS) - 1


# ---------------------------------------------------------------------------
# Packing / unpacking
# ---------------------------------------------------------------------------
def pack_indices(indices) -> torch.Tensor:
    """Pack a flat sequence of 9-bit indices, 7 per uint64 word.

    Host input (sequence / numpy / CPU tensor): packed by the library's host
    packer, returns a CPU ``torch.uint64`` tensor as the reference does
    (``lithe/kernels/packed.py:38-52``). A GPU tensor is packed on the GPU and
    the words stay on its device. Values outside [0, 511] raise ValueError.
    """
    lib = _hip.load()
    if isinstance(indices, torch.Tensor) and indices.is_cuda:
        flat = indices.reshape(-1).contiguous()
        if flat.dtype not in (torch.int16, torch.int32, torch.int64):
            flat = flat.to(torch.int32)
        n = flat.numel()
        words = torch.empty(-(-n // PER_WORD), dtype=torch.uint64, device=flat.device)
        err = torch.zeros(1, dtype=torch.int32, device=flat.device)
        _hip.check(lib.lithe_pack9(_hip.ptr(flat), _hip.dtype_code(flat.dtype), n, _hip.ptr(words),
                                   _hip.ptr(err), _hip.stream_of(flat.device)), "lithe_pack9")
        if int(err.item()):
            raise ValueError("indices must be < 512 for 9-bit packing")
        return words
    if isinstance(indices, torch.Tensor):
        indices = indices.numpy()
    flat = np.asarray(indices).reshape(-1)
    if flat.size and (int(flat.max()) > INDEX_MASK or int(flat.min()) < 0):
        raise ValueError("indices must be < 512 for 9-bit packing")
    flat16 = np.ascontiguousarray(flat, dtype=np.uint16)
    words = np.zeros(-(-flat16.size // PER_WORD), dtype=np.uint64)
    rc = lib.lithe_pack9_host(flat16.ctypes.data_as(ctypes.c_void_p), flat16.size,
                              words.ctypes.data_as(ctypes.c_void_p))
    _hip.check(rc, "pack_indices")
    return torch.from_numpy(words.view(np.int64)).view(torch.uint64)


def unpack_indices(words: torch.Tensor, n: int, dtype: torch.dtype = torch.int64) -> torch.Tensor:
    """Inverse of ``pack_indices`` on the GPU: (n,) int64 (lithe/kernels/packed.py:55-60)."""
    _hip.require_gpu(words)
    w = words.reshape(-1).contiguous()
    if n > w.numel() * PER_WORD:
        raise ValueError(f"{n} indices need {-(-n // PER_WORD)} words, got {w.numel()}")
    out = torch.empty(n, dtype=dtype, device=w.device)
    _hip.check(_hip.load().lithe_unpack9(_hip.ptr(w), n, _hip.ptr(out), _hip.dtype_code(dtype),
                                         _hip.stream_of(w.device)), "lithe_unpack9")
    return out


# ---------------------------------------------------------------------------
# Layout
# ---------------------------------------------------------------------------
@dataclass
class PackedLayout:
    """Where every module's A and B blocks sit in the packed stream of one adapter."""

    names: List[str]
    shapes_a: List[Tuple[int, int]]
    shapes_b: List[Tuple[int, int]]
    a_off: List[int]
    b_off: List[int]
    sides: torch.Tensor                     # (total_blocks,) int8, 0 = A block, 1 = B block
    num_levels: int
    block_size: int
    scaling: float                          # alpha / rank
    _sides_dev: Dict[str, torch.Tensor] = field(default_factory=dict, repr=False)
    _index: Dict[str, int] = field(default_factory=dict, repr=False)

    @property
    def total_blocks(self) -> int:
        return int(self.sides.numel())

    @property
    def num_indices(self) -> int:
        return self.total_blocks * self.num_levels

    @property
    def num_words(self) -> int:
        return (self.num_indices + PER_WORD - 1) // PER_WORD

    def sides_on(self, device) -> torch.Tensor:
        key = str(device)
        if key not in self._sides_dev:
            self._sides_dev[key] = self.sides.to(device).contiguous()
        return self._sides_dev[key]

    def module(self, name: str) -> Tuple[int, Tuple[int, int], Tuple[int, int], int, int]:
        """(position, shape_a, shape_b, a_off, b_off) of module ``name``."""
        if not self._index:
            self._index.update({n: i for i, n in enumerate(self.names)})
        i = self._index[name]
        return i, self.shapes_a[i], self.shapes_b[i], self.a_off[i], self.b_off[i]

    @classmethod
    def from_adapter(cls, ad) -> "PackedLayout":
        return cls.from_modules(ad.modules, ad.num_levels, ad.block_size, float(ad.alpha) / ad.rank)

    @classmethod
    def from_modules(cls, modules: Sequence[Dict], num_levels: int = 3, block_size: int = 64,
                     scaling: float = 1.0) -> "PackedLayout":
        """Layout of modules [{"name", "shape_a", "shape_b"}]: per module A blocks then B blocks."""
        names, sa, sb, a_off, b_off, parts = [], [], [], [], [], []
        cursor = 0
        for m in modules:
            n_a = quant.num_blocks(m["shape_a"], block_size)
            n_b = quant.num_blocks(m["shape_b"], block_size)
            names.append(m["name"])
            sa.append(tuple(int(s) for s in m["shape_a"]))
            sb.append(tuple(int(s) for s in m["shape_b"]))
            a_off.append(cursor)
            b_off.append(cursor + n_a)
            parts.append(np.concatenate([np.zeros(n_a, np.int8), np.ones(n_b, np.int8)]))
            cursor += n_a + n_b
        sides = torch.from_numpy(np.concatenate(parts) if parts else np.zeros(0, np.int8))
        return cls(names=names, shapes_a=sa, shapes_b=sb, a_off=a_off, b_off=b_off, sides=sides,
                   num_levels=int(num_levels), block_size=int(block_size), scaling=float(scaling))

    def ingest_table(self) -> torch.Tensor:
        """(2 * n_modules, 3) int64 segment table of ``lithe_ingest``: per factor in residency
        order, its first block, its block count and its first element in the ``.lithe`` stream."""
        key = "ingest_table"
        if key not in self._sides_dev:
            ba = np.array([quant.num_blocks(s, self.block_size) for s in self.shapes_a], np.int64)
            bb = np.array([quant.num_blocks(s, self.block_size) for s in self.shapes_b], np.int64)
            table = np.zeros((2 * len(self.names), 3), np.int64)
            rc = _hip.load().lithe_ingest_table(len(self.names), ba.ctypes.data_as(ctypes.c_void_p),
                                                bb.ctypes.data_as(ctypes.c_void_p), self.num_levels,
                                                table.ctypes.data_as(ctypes.c_void_p))
            _hip.check(rc, "lithe_ingest_table")
            self._sides_dev[key] = torch.from_numpy(table)
        return self._sides_dev[key]

    def table_on(self, device) -> torch.Tensor:
        """Device copy of ``ingest_table`` (read by the ingest and stacked-decode kernels)."""
        key = "table:" + str(device)
        if key not in self._sides_dev:
            self._sides_dev[key] = self.ingest_table().to(device)
        return self._sides_dev[key]

    def matches_modules(self, modules: Sequence[Dict], num_levels: int, block_size: int) -> bool:
        """True when ``modules`` ([{"name", "shape_a", "shape_b"}]) are this layout's, in order."""
        return (num_levels == self.num_levels and block_size == self.block_size and len(modules) == len(self.names)
                and all(m["name"] == n and tuple(m["shape_a"]) == a and tuple(m["shape_b"]) == b
                        for m, n, a, b in zip(modules, self.names, self.shapes_a, self.shapes_b)))

    def matches(self, ad) -> bool:
        return (len(ad.modules) == len(self.names)
                and all(m["name"] == n and tuple(m["shape_a"]) == a and tuple(m["shape_b"]) == b
                        for m, n, a, b in zip(ad.modules, self.names, self.shapes_a, self.shapes_b)))


def flat_indices(ad, layout: PackedLayout) -> np.ndarray:
    """The adapter's indices in packed-stream order: per module A blocks then B blocks,
    each block contributing its L indices (block, level)-major."""
    parts = []
    for name in layout.names:
        idx = ad.indices[name]
        parts.append(np.asarray(idx["A"]).T.reshape(-1))
        parts.append(np.asarray(idx["B"]).T.reshape(-1))
    return np.concatenate(parts).astype(np.uint16) if parts else np.zeros(0, np.uint16)


def blockify_factors(layout: PackedLayout, factors: Dict[str, Tuple[torch.Tensor, torch.Tensor]],
                     device) -> torch.Tensor:
    """Dense factors {module: (A (r, d_in), B (d_out, r))} -> (total_blocks, block_size) fp32 on
    ``device``: each factor row-major blockified at its layout offset, zero-padded to whole blocks
    (``lithe/quant.py:23-43`` per factor, in residency order). One concatenation builds it; zero
    runs appear only where a factor does not fill its last block."""
    bs = layout.block_size
    segs = []
    for name, sa, sb, ao, bo in zip(layout.names, layout.shapes_a, layout.shapes_b, layout.a_off, layout.b_off):
        if name not in factors:
            raise ValueError(f"missing factors of module {name}")
        a, b = factors[name]
        if tuple(a.shape) != sa or tuple(b.shape) != sb:
            raise ValueError(f"{name}: factors {tuple(a.shape)} / {tuple(b.shape)}, layout {sa} / {sb}")
        segs.append((ao * bs, a))
        segs.append((bo * bs, b))
    segs.sort(key=lambda s: s[0])
    total = layout.total_blocks * bs
    bounds = [(off, off + w.numel()) for off, w in segs] + [(total, total)]
    if any(nxt < end for (_, end), (nxt, _) in zip(bounds, bounds[1:])):
        raise ValueError("layout offsets overlap")
    gaps = [nxt - end for (_, end), (nxt, _) in zip([(0, 0)] + bounds, bounds)]
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    with torch.no_grad():    # no per-factor detach: nothing here is recorded for autograd
        zeros = torch.zeros(max(gaps), dtype=torch.float32, device=dev)
        parts = []
        for (_, w), gap in zip(segs + [(None, None)], gaps):
            if gap:
                parts.append(zeros[:gap])
            if w is not None:
                flat = w.reshape(-1)
                if flat.dtype != torch.float32 or flat.device != dev:
                    flat = flat.to(device=dev, dtype=torch.float32)
                parts.append(flat)
        out = torch.empty((layout.total_blocks, bs), dtype=torch.float32, device=dev)
        if parts:
            torch.cat(parts, out=out.view(-1))
    return out


def pack_adapter(ad, layout: Optional[PackedLayout] = None) -> Tuple[torch.Tensor, PackedLayout]:
    """(packed uint64 words on CPU, layout) for one ``LitheAdapter``."""
    if ad.n_bits != INDEX_BITS:
        raise ValueError(f"packing assumes 9-bit indices, adapter has n_bits={ad.n_bits}")
    layout = layout or PackedLayout.from_adapter(ad)
    if not layout.matches(ad):
        raise ValueError("adapter modules do not match the layout")
    return pack_indices(flat_indices(ad, layout)), layout


# ---------------------------------------------------------------------------
# Decode
# ---------------------------------------------------------------------------
def _check_pools(pool_a: torch.Tensor, pool_b: torch.Tensor, layout: PackedLayout):
    if pool_a.shape != pool_b.shape or pool_a.dim() != 3:
        raise ValueError("pools must both be (L, K, B)")
    if pool_a.shape[0] != layout.num_levels or pool_a.shape[2] != layout.block_size:
        raise ValueError("pool shape does not match the layout")
    if layout.block_size != 64:
        raise ValueError("lithe_amd decodes 64-value blocks only")


def _decode(src: _hip.IndexSrc, n_blocks: int, sides: Optional[torch.Tensor], pool_a, pool_b,
            out: torch.Tensor, slots: Optional[torch.Tensor] = None, n_sel: int = 1,
            out_sel_stride: int = 0) -> torch.Tensor:
    lut_a = _hip.lut_from_pools(pool_a, torch.float32)
    lut_b = _hip.lut_from_pools(pool_b, torch.float32)
    rc = _hip.load().lithe_decode(ctypes.byref(src), _hip.ptr(slots), n_sel, n_blocks, _hip.ptr(sides),
                                  ctypes.byref(lut_a), ctypes.byref(lut_b), _hip.ptr(out),
                                  _hip.dtype_code(out.dtype), out_sel_stride or n_blocks * 64, None,
                                  _hip.stream_of(out.device))
    _hip.check(rc, "lithe_decode")
    return out


def decode_packed(words: torch.Tensor, layout: PackedLayout, pool_a: torch.Tensor,
                  pool_b: torch.Tensor, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Decode every block of one packed adapter -> (total_blocks, block_size) on the GPU.

    ``dtype`` bf16 (the reference's kernel output) or float32. Pools are the fp32
    (L, K, B) pools of ``lithe_amd.codebook.build_pools``.
    """
    _check_pools(pool_a, pool_b, layout)
    _hip.require_gpu(words)
    if dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("decode_packed produces bfloat16 or float32")
    w = words.reshape(-1)
    if w.numel() < layout.num_words:
        raise ValueError("words shorter than the layout")
    out = torch.empty((layout.total_blocks, layout.block_size), dtype=dtype, device=w.device)
    if layout.total_blocks == 0:
        return out
    from ._delta import packed_source
    src = packed_source(w.contiguous(), layout.num_levels, 0)
    return _decode(src, layout.total_blocks, layout.sides_on(w.device), pool_a, pool_b, out)


def decode_packed_slots(bank: torch.Tensor, slots: torch.Tensor, layout: PackedLayout, pool_a: torch.Tensor,
                        pool_b: torch.Tensor, out: Optional[torch.Tensor] = None,
                        dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Decode the selected slots of a (n_slots, n_words) bank into (n_sel, total_blocks, 64) in one launch."""
    _check_pools(pool_a, pool_b, layout)
    _hip.require_gpu(bank, slots)
    if bank.dim() != 2 or bank.shape[1] < layout.num_words:
        raise ValueError("bank must be (n_slots, n_words >= layout.num_words)")
    sl = slots.reshape(-1).to(torch.int32).contiguous()
    n_sel = sl.numel()
    if out is None:
        out = torch.empty((n_sel, layout.total_blocks, layout.block_size), dtype=dtype, device=bank.device)
    if out.shape != (n_sel, layout.total_blocks, layout.block_size) or not out.is_contiguous():
        raise ValueError("out must be a contiguous (n_sel, total_blocks, 64) tensor")
    if n_sel == 0 or layout.total_blocks == 0:
        return out
    from ._delta import packed_source
    src = packed_source(bank, layout.num_levels, 0)
    return _decode(src, layout.total_blocks, layout.sides_on(bank.device), pool_a, pool_b, out,
                   slots=sl, n_sel=n_sel, out_sel_stride=layout.total_blocks * layout.block_size)


def decode_int16(idx: torch.Tensor, layout: PackedLayout, pool_a: torch.Tensor,
                 pool_b: torch.Tensor) -> torch.Tensor:
    """Same decode from an unpacked (total_blocks, L) int16 index tensor (residency A/B check)."""
    _check_pools(pool_a, pool_b, layout)
    _hip.require_gpu(idx)
    flat = idx.reshape(-1).to(torch.int16).contiguous()
    if flat.numel() != layout.num_indices:
        raise ValueError("idx must hold total_blocks * num_levels indices")
    out = torch.empty((layout.total_blocks, layout.block_size), dtype=torch.bfloat16, device=idx.device)
    if layout.total_blocks == 0:
        return out
    src = _hip.IndexSrc()
    src.base = flat.data_ptr()
    src.kind = _hip.IDX_BLOCK_I16
    src.num_levels = layout.num_levels
    src.slot_stride = flat.numel()
    src.level_stride = 0
    src.block_off = 0
    src.n_slots = 1
    return _decode(src, layout.total_blocks, layout.sides_on(idx.device), pool_a, pool_b, out)


def decode_packed_stacked(bank: torch.Tensor, slots: torch.Tensor, layout: PackedLayout, pool_a: torch.Tensor,
                          pool_b: torch.Tensor, out: Optional[torch.Tensor] = None,
                          dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Decode the selected slots of a (n_slots, n_words) bank in one launch into the stacked
    serving layout: a flat (n_sel * total_blocks * 64,) buffer in which every factor holds its
    selections side by side (``split_stacked`` gives the per-module (n_sel, r, d_in) and
    (n_sel, d_out, r) views that ``PerSampleLoRALinear`` would otherwise build with torch.stack)."""
    _check_pools(pool_a, pool_b, layout)
    _hip.require_gpu(bank, slots)
    if bank.dim() != 2 or bank.shape[1] < layout.num_words:
        raise ValueError("bank must be (n_slots, n_words >= layout.num_words)")
    sl = slots.reshape(-1).to(torch.int32).contiguous()
    n_sel = sl.numel()
    numel = n_sel * layout.total_blocks * layout.block_size
    if out is None:
        out = torch.empty(numel, dtype=dtype, device=bank.device)
    if out.numel() != numel or not out.is_contiguous() or out.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"out must be a contiguous bf16 / fp32 tensor of {numel} elements")
    if n_sel == 0 or layout.total_blocks == 0:
        return out
    from ._delta import packed_source
    src = packed_source(bank, layout.num_levels, 0)
    table = layout.table_on(bank.device)
    lut_a = _hip.lut_from_pools(pool_a, torch.float32)
    lut_b = _hip.lut_from_pools(pool_b, torch.float32)
    rc = _hip.load().lithe_decode_stacked(ctypes.byref(src), _hip.ptr(sl), n_sel, layout.total_blocks, table.shape[0],
                                          _hip.ptr(table), _hip.ptr(layout.sides_on(bank.device)),
                                          ctypes.byref(lut_a), ctypes.byref(lut_b), _hip.ptr(out),
                                          _hip.dtype_code(out.dtype), None, _hip.stream_of(out.device))
    _hip.check(rc, "lithe_decode_stacked")
    return out


def split_stacked(out: torch.Tensor, layout: PackedLayout, n_sel: int) -> Dict[str, Tuple[torch.Tensor, torch.Tensor]]:
    """name -> (A (n_sel, r, d_in), B (n_sel, d_out, r)) views of a ``decode_packed_stacked`` buffer.

    The factors lie back to back in residency order, so one ``split`` cuts every factor's
    chunk; the sizes and shapes are computed once per layout and selection count."""
    key = ("stacked_split", n_sel)
    plan = layout._sides_dev.get(key)
    if plan is None:
        bs = layout.block_size
        sizes, shapes, pos = [], [], 0
        for name, sa, sb, ao, bo in zip(layout.names, layout.shapes_a, layout.shapes_b, layout.a_off, layout.b_off):
            for shape, off in ((sa, ao), (sb, bo)):
                n = shape[0] * shape[1]
                nb = quant.num_blocks(shape, bs)
                if n != nb * bs:
                    raise ValueError(f"{name}: factors that do not fill whole blocks have no stacked view")
                if off * bs != pos:
                    raise ValueError("stacked views need the layout's factors back to back in residency order")
                sizes.append(n_sel * n)
                shapes.append((n_sel, shape[0], shape[1]))
                pos += n
        plan = (sizes, shapes, n_sel * pos)
        layout._sides_dev[key] = plan
    sizes, shapes, total = plan
    chunks = out.reshape(-1)[:total].split(sizes)
    return {name: (chunks[2 * i].view(shapes[2 * i]), chunks[2 * i + 1].view(shapes[2 * i + 1]))
            for i, name in enumerate(layout.names)}


def split_decoded(out: torch.Tensor, layout: PackedLayout) -> Dict[str, Tuple[torch.Tensor, torch.Tensor]]:
    """name -> (A (r, d_in), B (d_out, r)) as views into the decode output (one ``split`` of the
    flat output into factor chunks and block padding, computed once per layout)."""
    key = "decoded_split"
    plan = layout._sides_dev.get(key)
    if plan is None:
        bs = layout.block_size
        segs = []
        for sa, sb, ao, bo in zip(layout.shapes_a, layout.shapes_b, layout.a_off, layout.b_off):
            segs += [(ao * bs, sa), (bo * bs, sb)]
        order = sorted(range(len(segs)), key=lambda i: segs[i][0])
        sizes, where, pos = [], [0] * len(segs), 0
        for i in order:
            off, shape = segs[i]
            if off < pos:
                raise ValueError("layout offsets overlap")
            if off > pos:
                sizes.append(off - pos)              # padding of the previous factor's last block
            where[i] = len(sizes)
            sizes.append(shape[0] * shape[1])
            pos = off + shape[0] * shape[1]
        plan = (sizes, where, [tuple(sh) for _, sh in segs], pos)
        layout._sides_dev[key] = plan
    sizes, where, shapes, total = plan
    chunks = out.reshape(-1)[:total].split(sizes)
    return {name: (chunks[where[2 * i]].view(shapes[2 * i]), chunks[where[2 * i + 1]].view(shapes[2 * i + 1]))
            for i, name in enumerate(layout.names)}


def decode_factors(ad, device="cuda", dtype: torch.dtype = torch.float32) -> Dict[str, Tuple[torch.Tensor, torch.Tensor]]:
    """Every factor of an index adapter decoded on the GPU: {module: (A (r, d_in), B (d_out, r))}.

    The adapter is packed in its own layout, every block decoded in one launch (``dtype`` fp32:
    the reference's fp32 decode, ``lithe/quant.py:74-92``, bit for bit) and the result split
    into per-module views of one buffer."""
    from .. import codebook as cb
    words, layout = pack_adapter(ad)
    pools = (cb.build_pools(ad.sigma_a, ad.block_size, ad.n_bits).to(device),
             cb.build_pools(ad.sigma_b, ad.block_size, ad.n_bits).to(device))
    out = decode_packed(words.view(torch.int64).to(device), layout, *pools, dtype=dtype)
    return split_decoded(out, layout)
