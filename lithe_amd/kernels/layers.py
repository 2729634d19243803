"""Linear wrappers that route every sample of a batch to its own adapter.

API of ``lithe/kernels/layers.py``:

``PerSampleLoRALinear``  decoded factors (A, B, scale) per adapter slot.
``IndexLoRALinear``      index-resident slots; the delta is decoded inside the
                         shrink / expand tiles and accumulated into the base
                         output in the same pass (``y = base(x)`` then
                         ``y += delta`` with the rounding of ``out + delta``).
                         ``IndexLoRALinear.from_bank`` reads the slots straight
                         from a bit-packed ``PackedBank``.

Routing: with ``assign`` unset, ``IndexLoRALinear`` uses slot 0 for every
sample and ``PerSampleLoRALinear`` uses slot ``i % n_slots``; otherwise
``assign`` (B,) gives the slot of every sample. All deltas run on the GPU.
"""
from __future__ import annotations

from typing import Callable, Dict, Iterable, List, Optional, Sequence, Tuple

import torch
from torch import nn

from . import _delta, _hip
from . import ops as _ops  # noqa: F401  (registers the lithe_amd:: operators)
from .sgmv import lora_delta_dense, per_sample_lora_delta

Factor = Tuple[torch.Tensor, torch.Tensor, float]


class PerSampleLoRALinear(nn.Module):
    """y = W x + scale_j * B_j A_j x for the slot j of every sample (decoded factors)."""

    def __init__(self, base: nn.Linear, kernel: str = "sgmv"):
        super().__init__()
        if kernel not in ("sgmv", "loop"):
            raise ValueError(f"kernel must be 'sgmv' or 'loop', got {kernel!r}")
        self.base = base
        for p in self.base.parameters():
            p.requires_grad_(False)
        self.kernel = kernel          # both names run the same HIP kernels
        self.factors: List[Factor] = []
        self.per_sample = False
        self.assign: Optional[torch.Tensor] = None
        self._stacked = None

    def set_factors(self, factors: Sequence[Factor], per_sample: bool = True) -> None:
        """Install slot factors by reference (no copy); stacking happens lazily in forward."""
        self.factors = list(factors)
        self.per_sample = per_sample
        self._stacked = None

    def set_stacked(self, a: torch.Tensor, b: torch.Tensor, scales: torch.Tensor) -> None:
        """Install already stacked factors a (n, r, d_in), b (n, d_out, r) and scales (n,) -- e.g.
        views from ``PackedBank.decode_stacked`` -- without the stacking copy."""
        if a.dim() != 3 or b.dim() != 3 or a.shape[0] != b.shape[0] or scales.numel() != a.shape[0]:
            raise ValueError("stacked factors must be (n, r, d_in), (n, d_out, r) with n scales")
        self.factors = [(a[i], b[i], float(scales[i])) for i in range(a.shape[0])]
        self.per_sample = True
        self._stacked = (a.contiguous(), b.contiguous(), scales.to(device=a.device, dtype=torch.float32))

    def clear(self) -> None:
        self.set_factors([], per_sample=False)

    def _slots(self, bsz: int, device) -> torch.Tensor:
        if self.assign is not None:
            return self.assign.to(device=device, dtype=torch.int32)
        return (torch.arange(bsz, device=device) % len(self.factors)).to(torch.int32)

    def _build_stacked(self):
        if self._stacked is None:
            a = torch.stack([f[0] for f in self.factors]).contiguous()
            b = torch.stack([f[1] for f in self.factors]).contiguous()
            s = torch.tensor([float(f[2]) for f in self.factors], dtype=torch.float32, device=a.device)
            self._stacked = (a, b, s)
        return self._stacked

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = self.base(x)
        if not self.factors:
            return out
        squeeze = x.dim() == 2
        if x.dim() not in (2, 3):
            raise ValueError(f"unsupported input rank {x.dim()}")
        x3 = x.unsqueeze(1) if squeeze else x
        out3 = out.unsqueeze(1) if squeeze else out
        bsz = x3.shape[0]
        if not self.per_sample:
            a, b, s = self.factors[0]
            sc = torch.full((bsz,), float(s), dtype=torch.float32, device=x.device)
            lora_delta_dense(x3, a.unsqueeze(0), b.unsqueeze(0), sc, base=out3,
                             slots=torch.zeros(bsz, dtype=torch.int32, device=x.device), bmm_semantics=True)
            return out
        a, b, s = self._build_stacked()
        idx = self._slots(bsz, x.device)
        scale = s.index_select(0, idx.long()).to(x.dtype).float()
        # bf16 3-D input takes the kernel semantics of the reference (scale on mid);
        # 2-D modulation inputs and fp32 take its bmm semantics (scale on the delta).
        bmm = squeeze or x.dtype != torch.bfloat16
        lora_delta_dense(x3, a, b, scale, base=out3, slots=idx, bmm_semantics=bmm)
        return out


class IndexLoRALinear(nn.Module):
    """y = W x + per-sample delta decoded on the fly from resident index slots."""

    def __init__(self, base: nn.Linear, idx_a: torch.Tensor, idx_b: torch.Tensor,
                 pool_a: torch.Tensor, pool_b: torch.Tensor, rank: int, scaling: float):
        super().__init__()
        self.base = base
        for p in self.base.parameters():
            p.requires_grad_(False)
        # (n_slots, L, n_blocks) int32; pools (L, K, block) in the activation dtype
        self.register_buffer("idx_a", idx_a.to(torch.int32), persistent=False)
        self.register_buffer("idx_b", idx_b.to(torch.int32), persistent=False)
        self.register_buffer("pool_a", pool_a, persistent=False)
        self.register_buffer("pool_b", pool_b, persistent=False)
        self.rank = int(rank)
        self.d_out = base.out_features
        self.scaling = float(scaling)
        self.assign: Optional[torch.Tensor] = None
        self._bank = None          # (PackedBank, a_off, b_off) for bank-backed layers

    @classmethod
    def from_bank(cls, base: nn.Linear, bank, name: str, dtype: Optional[torch.dtype] = None) -> "IndexLoRALinear":
        """Layer whose slots are read from the packed ``bank`` (module ``name`` of its layout)."""
        _, sa, sb, a_off, b_off = bank.layout.module(name)
        if sa[1] != base.in_features or sb[0] != base.out_features:
            raise ValueError(f"{name}: layout shapes {sa}/{sb} do not match the linear")
        dtype = dtype or base.weight.dtype
        empty = torch.zeros(0, bank.layout.num_levels, 0, dtype=torch.int32, device=bank.device)
        layer = cls(base, empty, empty, bank.pool_a.to(dtype), bank.pool_b.to(dtype), sa[0], bank.layout.scaling)
        layer._bank = (bank, a_off, b_off)
        return layer

    @property
    def num_slots(self) -> int:
        return int(self._bank[0].num_slots if self._bank else self.idx_a.shape[0])

    def _factors(self, dtype: torch.dtype):
        lut_a = _hip.lut_from_pools(self.pool_a, dtype)
        lut_b = _hip.lut_from_pools(self.pool_b, dtype)
        L = int(self.pool_a.shape[0])
        if self._bank is not None:
            bank, a_off, b_off = self._bank
            words = bank.words
            return _delta.indexed_factors(_delta.packed_source(words, L, a_off),
                                          _delta.packed_source(words, L, b_off), lut_a, lut_b)
        d_in = self.base.in_features
        return _delta.indexed_factors(_delta.index_source(self.idx_a, L, self.rank * d_in // 64),
                                      _delta.index_source(self.idx_b, L, self.d_out * self.rank // 64),
                                      lut_a, lut_b)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = self.base(x)
        squeeze = x.dim() == 2
        x3 = x.unsqueeze(1) if squeeze else x
        out3 = out.unsqueeze(1) if squeeze else out
        if x3.dim() != 3:
            raise ValueError(f"unsupported input rank {x.dim()}")
        _hip.require_gpu(x3)
        if x.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError(f"lithe_amd kernels take bfloat16 or float32 activations, got {x.dtype}")
        bsz = x3.shape[0]
        assign = self.assign
        if assign is None:
            slots = torch.zeros((bsz, 1), dtype=torch.int32, device=x.device)
        else:
            if assign.shape != (bsz,):
                raise ValueError(f"assign must be ({bsz},)")
            slots = assign.to(device=x.device, dtype=torch.int32).reshape(-1, 1).contiguous()
        if not out3.is_contiguous():
            out3 = out3.contiguous()
            out = out3.squeeze(1) if squeeze else out3
        # through the torch.library ops (lithe_amd/kernels/ops.py): one opaque in-place op for
        # torch.compile / FX
        if self._bank is not None:
            bank, a_off, b_off = self._bank
            torch.ops.lithe_amd.bank_lora_delta_(x3.contiguous(), out3, bank.words, a_off, b_off, self.pool_a,
                                                 self.pool_b, slots, self.rank, self.scaling)
        else:
            torch.ops.lithe_amd.index_lora_delta_(x3.contiguous(), out3, self.idx_a, self.idx_b, self.pool_a,
                                                  self.pool_b, slots, self.rank, self.scaling)
        return out


def wrap_linears(model: nn.Module, paths: Iterable[str],
                 factory: Callable[[str, nn.Linear], nn.Module]) -> Dict[str, nn.Module]:
    """Replace ``model.<path>`` (an ``nn.Linear``) by ``factory(path, linear)`` for every path."""
    wrapped = {}
    for path in paths:
        base = model.get_submodule(path)
        if not isinstance(base, nn.Linear):
            raise TypeError(f"{path} is not nn.Linear")
        parent_name, _, child = path.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        module = factory(path, base)
        setattr(parent, child, module)
        wrapped[path] = module
    return wrapped


__all__ = ["IndexLoRALinear", "PerSampleLoRALinear", "wrap_linears", "per_sample_lora_delta"]
