"""GPU-resident bank of bit-packed adapters (API of ``PackedBank``, ``serving/_common.py:211-255``).

All slots share one ``PackedLayout`` and one pair of fp32 pools. Where the
reference keeps a Python list of per-slot tensors, this bank is one
contiguous (capacity, n_words) uint64 tensor: a slot id is a row, any kernel
can address every slot through one pointer, and a 10,000-slot bank of the
342-linear FLUX layout is a single 24.0 GB allocation.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import torch

from .. import codebook as cb
from . import _hip
from .packed import PackedLayout, decode_packed_slots, pack_adapter, split_decoded


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
        if capacity <= self._words.shape[0]:
            return
        grown = torch.zeros((capacity, self.layout.num_words), dtype=torch.int64, device=self.device)
        grown[: self.num_slots].copy_(self._words[: self.num_slots])
        self._words = grown

    def add(self, words: torch.Tensor) -> int:
        """Append one adapter's packed words (CPU or GPU); returns its slot id."""
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
        if n <= self.num_slots:
            return
        self.reserve(n)
        self._words[self.num_slots:n].copy_(self._words[template_slot].expand(n - self.num_slots, -1))
        self.num_slots = n

    def fill_random(self, n: int, generator: Optional[torch.Generator] = None) -> None:
        """Grow to ``n`` slots of uniformly random 9-bit fields (padding fields of the last word zero)."""
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

    def decode_diffusers(self, slot: int) -> Dict[str, Tuple[torch.Tensor, torch.Tensor, float]]:
        s = self.layout.scaling
        return {k: (a, b, s) for k, (a, b) in self.decode(slot).items()}

    @property
    def slot_bytes(self) -> int:
        return self.layout.num_words * 8
