"""GPU-resident bank of bit-packed adapters (API of ``PackedBank``, ``serving/_common.py:211-255``).

All slots share one ``PackedLayout`` and one pair of fp32 pools. Where the
reference keeps a Python list of per-slot tensors, this bank is one
contiguous (capacity, n_words) uint64 tensor: a slot id is a row, any kernel
can address every slot through one pointer, and a 10,000-slot bank of the
342-linear FLUX layout is a single 24.0 GB allocation.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from .. import codebook as cb
from . import _hip
from .packed import (PackedLayout, blockify_factors, decode_packed_slots, decode_packed_stacked, pack_adapter, split_decoded,
                     split_stacked)


class PackedBank:
    """Resident 9-bit packed index slots sharing one layout and one pair of fp32 pools."""

    def __init__(self, layout: PackedLayout, device, capacity: int = 16,
                 pools: Optional[Tuple[torch.Tensor, torch.Tensor]] = None):
        self.layout = layout
        self.device = torch.device(device)
        if pools is None:
            pools = cb.twin_pools()
        self.pool_a, self.pool_b = (p.to(self.device) for p in pools)
        layout.sides_on(self.device)
        # int64 storage (torch has more kernels for it); the bits are the uint64 words.
        self._words = torch.zeros((max(1, int(capacity)), layout.num_words), dtype=torch.int64, device=self.device)
        self.num_slots = 0
        self.generation = 0                # bumped by every write into the words (cached results are stale)
        self._free: List[int] = []        # freed slot ids, ascending
        self._stage = None                 # (pinned stream, device stream, error word, copy event)

    # -------------------------------------------------------------- construction
    @classmethod
    def from_adapters(cls, ads, device) -> Tuple["PackedBank", List[torch.Tensor]]:
        """Bank with the layout of ``ads[0]`` (empty) plus every adapter's packed CPU words."""
        words0, layout = pack_adapter(ads[0])
        pools = (cb.build_pools(ads[0].sigma_a, ads[0].block_size, ads[0].n_bits),
                 cb.build_pools(ads[0].sigma_b, ads[0].block_size, ads[0].n_bits))
        bank = cls(layout, device, capacity=len(ads), pools=pools)
        cpu_words = [words0] + [pack_adapter(ad, layout)[0] for ad in ads[1:]]
        return bank, cpu_words

    @property
    def words(self) -> torch.Tensor:
        """(num_slots, n_words) view of the resident slots."""
        return self._words[: max(1, self.num_slots)]

    @property
    def slots(self) -> List[torch.Tensor]:
        """Per-slot views (the reference's list of slot tensors)."""
        return [self._words[i].view(torch.uint64) for i in range(self.num_slots)]

    def reserve(self, capacity: int) -> None:
        self.generation += 1
        if capacity <= self._words.shape[0]:
            return
        grown = torch.zeros((capacity, self.layout.num_words), dtype=torch.int64, device=self.device)
        grown[: self.num_slots].copy_(self._words[: self.num_slots])
        self._words = grown

    def add(self, words: torch.Tensor) -> int:
        """Append one adapter's packed words (CPU or GPU); returns its slot id."""
        self.generation += 1
        if words.numel() != self.layout.num_words:
            raise ValueError(f"expected {self.layout.num_words} words, got {words.numel()}")
        if self.num_slots == self._words.shape[0]:
            self.reserve(max(16, 2 * self.num_slots))
        w = words.reshape(-1)
        if w.dtype == torch.uint64:
            w = w.view(torch.int64)
        self._words[self.num_slots].copy_(w)
        self.num_slots += 1
        return self.num_slots - 1

    def fill_to(self, n: int, template_slot: int = 0) -> None:
        """Grow to ``n`` slots by copying a resident slot (distinct rows, same content)."""
        self.generation += 1
        if n <= self.num_slots:
            return
        self.reserve(n)
        self._words[self.num_slots:n].copy_(self._words[template_slot].expand(n - self.num_slots, -1))
        self.num_slots = n

    def fill_random(self, n: int, generator: Optional[torch.Generator] = None) -> None:
        """Grow to ``n`` slots of uniformly random 9-bit fields (padding fields of the last word zero)."""
        self.generation += 1
        self.reserve(n)
        k = n - self.num_slots
        if k <= 0:
            return
        nw = self.layout.num_words
        lo = self.num_slots
        chunk = max(1, (1 << 28) // nw)
        for s in range(lo, n, chunk):
            e = min(n, s + chunk)
            r = torch.randint(0, 1 << 62, (e - s, nw), dtype=torch.int64, device=self.device, generator=generator)
            r = (r << 1) | torch.randint(0, 2, (e - s, nw), dtype=torch.int64, device=self.device, generator=generator)
            r &= (1 << 63) - 1
            used = self.layout.num_indices - (nw - 1) * 7
            if used < 7:
                r[:, -1] &= (1 << (9 * used)) - 1
            self._words[s:e].copy_(r)
        self.num_slots = n

    def shrink_to(self, n: int) -> None:
        self.num_slots = min(self.num_slots, max(0, n))
        self._free = [f for f in self._free if f < self.num_slots]

    # -------------------------------------------------------------- slot allocation
    def alloc(self) -> int:
        """A slot id to load an adapter into: the lowest freed slot, else a new one at the end."""
        if self._free:
            return self._free.pop(0)
        if self.num_slots == self._words.shape[0]:
            self.reserve(max(16, 2 * self.num_slots))
        self.num_slots += 1
        return self.num_slots - 1

    def free(self, slot: int) -> None:
        """Return ``slot`` to the allocator. Its words stay until the slot is reloaded; routing a
        sample to a freed slot is the caller's error, as indexing a dropped list entry is in the
        reference's bank."""
        if not 0 <= slot < self.num_slots:
            raise IndexError(f"slot {slot} is not resident")
        if slot in self._free:
            raise ValueError(f"slot {slot} is already free")
        self._free.append(slot)
        self._free.sort()

    @property
    def num_free(self) -> int:
        return len(self._free)

    # -------------------------------------------------------------- ingest
    def _target(self, slot: Optional[int]) -> int:
        self.generation += 1
        if slot is None:
            return self.alloc()
        if not 0 <= slot < self.num_slots:
            raise IndexError(f"slot {slot} is not resident (bank has {self.num_slots})")
        if slot in self._free:
            self._free.remove(slot)
        return slot

    def _staging(self, n: int):
        """Pinned host and device buffers for one uint16 index stream, reused across loads."""
        st = self._stage
        if st is None or st[0].numel() < n:
            pin = torch.empty(n, dtype=torch.int16, pin_memory=True)
            dev = torch.empty(n, dtype=torch.int16, device=self.device)
            err = torch.zeros(1, dtype=torch.int32, device=self.device)
            st = (pin, dev, err, torch.cuda.Event())
            self._stage = st
        return st

    def load_stream(self, stream, slot: Optional[int] = None, on_device: bool = True) -> int:
        """Load one adapter from its ``.lithe`` index stream (uint16: the A matrices of every
        module, then the B matrices) into a slot; returns the slot id.

        ``on_device``: the stream is copied to the GPU and reordered + packed there straight into
        the slot (``lithe_ingest``); otherwise the host packer builds the words
        (``lithe_ingest_host``) and they are copied into the slot. Values above 511 raise
        ValueError before anything is written. Asynchronous on the current stream.
        """
        arr = np.ascontiguousarray(np.asarray(stream).reshape(-1)).view(np.uint16) if not isinstance(
            stream, torch.Tensor) else stream.reshape(-1).contiguous().cpu().numpy().view(np.uint16)
        lay = self.layout
        if arr.size != lay.num_indices:
            raise ValueError(f"stream holds {arr.size} indices, the layout needs {lay.num_indices}")
        if arr.size and int(arr.max()) > 511:
            raise ValueError("indices must be < 512 for 9-bit packing")
        table = lay.ingest_table()
        target = self._target(slot)
        row = self._words[target]
        lib = _hip.load()
        if on_device:
            pin, dev, err, ev = self._staging(arr.size)
            ev.synchronize()                        # the previous load's copy has left the pinned buffer
            pin[: arr.size].numpy()[:] = arr.view(np.int16)
            dev[: arr.size].copy_(pin[: arr.size], non_blocking=True)
            ev.record()
            tdev = lay.table_on(self.device)
            rc = lib.lithe_ingest(_hip.ptr(dev), arr.size, lay.num_levels, table.shape[0], _hip.ptr(tdev),
                                  _hip.ptr(row), lay.num_words, _hip.ptr(err), _hip.stream_of(self.device))
            _hip.check(rc, "lithe_ingest")
        else:
            words = np.empty(lay.num_words, np.uint64)
            rc = lib.lithe_ingest_host(arr.ctypes.data_as(ctypes.c_void_p), arr.size, lay.num_levels, table.shape[0],
                                       table.numpy().ctypes.data_as(ctypes.c_void_p),
                                       words.ctypes.data_as(ctypes.c_void_p), lay.num_words)
            _hip.check(rc, "lithe_ingest_host")
            row.copy_(torch.from_numpy(words.view(np.int64)))
        return target

    def load_lithe(self, path, slot: Optional[int] = None, verify: bool = True, on_device: bool = True) -> int:
        """Cold swap from a ``.lithe`` file (``lithe/fileio.py:119-152`` then ``pack_adapter``,
        ``lithe/kernels/packed.py:136-143``): read and check the file, then ``load_stream``.
        The file's modules, levels and block size must be the bank's layout."""
        from ..fileio import read_stream
        header, stream = read_stream(path, verify)
        book = header["codebook"]
        if not self.layout.matches_modules(header["modules"], int(book["num_levels"]), int(book["block_size"])):
            raise ValueError(f"{path}: modules do not match the bank layout")
        if int(book["n_bits"]) != 9:
            raise ValueError(f"{path}: the bank holds 9-bit indices, the file has n_bits={book['n_bits']}")
        return self.load_stream(stream, slot, on_device)

    def load_blob(self, path, slot: Optional[int] = None) -> int:
        """Cold swap from a raw index blob on disk: int16 indices already in the residency order
        (``flat_indices(ad, layout).astype(np.int16).tofile(path)``, the blob of
        ``serving/bench_hotswap.py:100-104``), packed on the GPU straight into the slot."""
        lay = self.layout
        arr = np.fromfile(path, dtype=np.int16)
        if arr.size != lay.num_indices:
            raise ValueError(f"{path}: {arr.size} indices, the layout needs {lay.num_indices}")
        if arr.size and (int(arr.max()) > 511 or int(arr.min()) < 0):
            raise ValueError("indices must be in [0, 511] for 9-bit packing")
        target = self._target(slot)
        pin, dev, err, ev = self._staging(arr.size)
        ev.synchronize()
        pin[: arr.size].numpy()[:] = arr
        dev[: arr.size].copy_(pin[: arr.size], non_blocking=True)
        ev.record()
        rc = _hip.load().lithe_pack9(_hip.ptr(dev), _hip.DT_I16, arr.size, _hip.ptr(self._words[target]),
                                     _hip.ptr(err), _hip.stream_of(self.device))
        _hip.check(rc, "lithe_pack9")
        return target

    def encode_factors(self, factors: Dict[str, Tuple[torch.Tensor, torch.Tensor]], slot: Optional[int] = None) -> int:
        """GPU re-quantisation of a dense adapter into a slot: ``factors`` {module: (A (r, d_in),
        B (d_out, r))} of this layout are blockified (row-major, zero-padded), encoded level by
        level with the closed-form search against the bank's fp32 pools (``lithe_encode``; A
        blocks with pool A, B blocks with pool B) straight into the residency order, and packed
        into the slot (``lithe_pack9``). Replaces ``quant.encode`` per factor +
        ``pack_adapter`` + ``PackedBank.add`` (``lithe/quant.py:84-88``,
        ``lithe/kernels/packed.py:136-143``). Returns the slot id."""
        lay = self.layout
        bs = lay.block_size
        blocks = blockify_factors(lay, factors, self.device)
        L = lay.num_levels
        idx = torch.empty(lay.total_blocks * L, dtype=torch.int16, device=self.device)
        lut_a = _hip.lut_from_pools(self.pool_a, torch.float32)
        lut_b = _hip.lut_from_pools(self.pool_b, torch.float32)
        lib = _hip.load()
        st = _hip.stream_of(self.device)
        _hip.check(lib.lithe_encode(_hip.ptr(blocks), lay.total_blocks, _hip.ptr(lay.sides_on(self.device)),
                                    ctypes.byref(lut_a), ctypes.byref(lut_b), _hip.ptr(idx), _hip.DT_I16, 1, L, None,
                                    st), "lithe_encode")
        target = self._target(slot)
        _, _, err, _ = self._staging(1)
        _hip.check(lib.lithe_pack9(_hip.ptr(idx), _hip.DT_I16, idx.numel(), _hip.ptr(self._words[target]),
                                   _hip.ptr(err), st), "lithe_pack9")
        return target

    def ingest_errors(self, clear: bool = True) -> int:
        """Error bits the device ingest recorded since the last clear (synchronises)."""
        st = self._stage
        if st is None:
            return 0
        v = int(st[2].item())
        if clear and v:
            st[2].zero_()
        return v

    # -------------------------------------------------------------- decode
    def decode(self, slot: int) -> Dict[str, Tuple[torch.Tensor, torch.Tensor]]:
        """Fused decode of one slot -> {module name: (A, B)} bf16 views."""
        out = self.decode_slots(torch.tensor([slot], dtype=torch.int32, device=self.device))
        return split_decoded(out[0], self.layout)

    def decode_slots(self, slots: torch.Tensor, out: Optional[torch.Tensor] = None,
                     dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """Decode several slots in one launch -> (n_sel, total_blocks, 64)."""
        if self.num_slots == 0:
            raise ValueError("bank is empty")
        return decode_packed_slots(self.words, slots, self.layout, self.pool_a, self.pool_b, out=out, dtype=dtype)

    def decode_stacked(self, slots, out: Optional[torch.Tensor] = None, dtype: torch.dtype = torch.bfloat16
                       ) -> Dict[str, Tuple[torch.Tensor, torch.Tensor]]:
        """Decode-on-swap for decoded-mode serving: the selected slots decoded in one launch to
        {module: (A (n, r, d_in), B (n, d_out, r))} views of one buffer (selection i = slots[i]),
        the stacked factors ``PerSampleLoRALinear`` and ``per_sample_lora_delta`` take."""
        sl = torch.as_tensor(slots, dtype=torch.int32).reshape(-1).to(self.device)
        if self.num_slots == 0:
            raise ValueError("bank is empty")
        buf = decode_packed_stacked(self.words, sl, self.layout, self.pool_a, self.pool_b, out=out, dtype=dtype)
        return split_stacked(buf, self.layout, sl.numel())

    def decode_diffusers(self, slot: int) -> Dict[str, Tuple[torch.Tensor, torch.Tensor, float]]:
        s = self.layout.scaling
        return {k: (a, b, s) for k, (a, b) in self.decode(slot).items()}

    @property
    def slot_bytes(self) -> int:
        return self.layout.num_words * 8
