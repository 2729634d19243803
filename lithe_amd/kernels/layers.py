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


def replace_module(model: nn.Module, path: str, new: nn.Module) -> nn.Module:
    """Put ``new`` at ``model.<path>`` (dotted, ModuleList indices included) and return the module
    it replaces."""
    owner_path, _, attr = path.rpartition(".")
    owner = model.get_submodule(owner_path) if owner_path else model
    old = getattr(owner, attr)
    setattr(owner, attr, new)
    return old


def _stack_factors(factors: Sequence[Factor]):
    """(A (n, r, d_in), B (n, d_out, r), scales (n,) fp32) of slot factors of one shape and device."""
    a0, b0, _ = factors[0]
    for a, b, _ in factors:
        if a.shape != a0.shape or b.shape != b0.shape or a.device != a0.device or b.device != a0.device:
            raise ValueError(f"slot factors must share one shape and device; got {tuple(a.shape)} / {tuple(b.shape)} "
                             f"after {tuple(a0.shape)} / {tuple(b0.shape)}")
    scales = torch.tensor([float(s) for _, _, s in factors], dtype=torch.float32, device=a0.device)
    return torch.stack([a for a, _, _ in factors]), torch.stack([b for _, b, _ in factors]), scales


class PerSampleLoRALinear(nn.Module):
    """y = W x + scale_j * B_j A_j x for the slot j of every sample (decoded factors).

    ``factors`` holds the slot factors as installed (A (r, d_in), B (d_out, r), scale); the
    kernels read them stacked, which is built once on the first forward after a change (or
    installed directly by ``set_stacked``). ``kernel`` is kept for the reference's API: "sgmv"
    and "loop" run the same HIP kernels.
    """

    def __init__(self, base: nn.Linear, kernel: str = "sgmv"):
        super().__init__()
        if kernel not in ("sgmv", "loop"):
            raise ValueError(f"kernel must be 'sgmv' or 'loop', got {kernel!r}")
        base.requires_grad_(False)
        self.base = base
        self.kernel = kernel
        self.assign: Optional[torch.Tensor] = None
        self.clear()

    def set_factors(self, factors: Sequence[Factor], per_sample: bool = True) -> None:
        """Install slot factors by reference (no copy); stacking happens lazily in forward."""
        self.factors: List[Factor] = list(factors)
        self.per_sample = per_sample
        self._stacked = None

    def clear(self) -> None:
        self.set_factors((), per_sample=False)

    def set_stacked(self, a: torch.Tensor, b: torch.Tensor, scales: torch.Tensor) -> None:
        """Install already stacked factors a (n, r, d_in), b (n, d_out, r) and scales (n,) -- e.g.
        views from ``PackedBank.decode_stacked`` -- without the stacking copy."""
        if a.dim() != 3 or b.dim() != 3 or a.shape[0] != b.shape[0] or scales.numel() != a.shape[0]:
            raise ValueError("stacked factors must be (n, r, d_in), (n, d_out, r) with n scales")
        self.factors = [(a[i], b[i], float(scales[i])) for i in range(a.shape[0])]
        self.per_sample = True
        self._stacked = (a.contiguous(), b.contiguous(), scales.to(device=a.device, dtype=torch.float32))

    def _slots(self, bsz: int, device) -> torch.Tensor:
        if self.assign is not None:
            return self.assign.to(device=device, dtype=torch.int32)
        return (torch.arange(bsz, device=device) % len(self.factors)).to(torch.int32)

    def _build_stacked(self):
        if self._stacked is None:
            self._stacked = _stack_factors(self.factors)
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
    """y = W x + per-sample delta decoded on the fly from resident index slots.

    ``idx_a`` (n_slots, L, rank * d_in / 64) and ``idx_b`` (n_slots, L, d_out * rank / 64) are the
    level-major indices of every slot (int16 and int32 are read as given, other integer dtypes
    are converted to int32); ``pool_a`` / ``pool_b`` (L, 512, 64) are in the activation dtype.
    """

    def __init__(self, base: nn.Linear, idx_a: torch.Tensor, idx_b: torch.Tensor,
                 pool_a: torch.Tensor, pool_b: torch.Tensor, rank: int, scaling: float):
        super().__init__()
        base.requires_grad_(False)
        self.base = base
        self.rank = int(rank)
        self.d_out = base.out_features
        self.scaling = float(scaling)
        self.assign: Optional[torch.Tensor] = None
        self._bank = None          # (PackedBank, a_off, b_off) for bank-backed layers
        self._eager = None         # (key, factors, route) of the last eager call
        idx = {}
        for name, t, blocks in (("idx_a", idx_a, -(-self.rank * base.in_features // 64)),
                                ("idx_b", idx_b, -(-self.d_out * self.rank // 64))):
            if t.dtype not in (torch.int16, torch.int32):
                t = t.to(torch.int32)
            if t.numel() and (t.dim() != 3 or t.shape[1] != pool_a.shape[0] or t.shape[2] != blocks):
                raise ValueError(f"{name} must be (n_slots, {pool_a.shape[0]}, {blocks}), got {tuple(t.shape)}")
            idx[name] = t
        for name, t in (("idx_a", idx["idx_a"]), ("idx_b", idx["idx_b"]), ("pool_a", pool_a), ("pool_b", pool_b)):
            self.register_buffer(name, t, persistent=False)

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
            if assign.dtype == torch.int32 and assign.device == x.device and assign.is_contiguous():
                slots = assign.view(-1, 1)
            else:
                slots = assign.to(device=x.device, dtype=torch.int32).reshape(-1, 1).contiguous()
        if not out3.is_contiguous():
            out3 = out3.contiguous()
            out = out3.squeeze(1) if squeeze else out3
        if not torch.compiler.is_compiling():
            # eager: the operator's body without the dispatcher, with the call descriptors kept
            # while the factors, tables and slot tensor stay the same (the kernels read the slot
            # values at launch, so an in-place update of assign needs no new descriptor). A bank's
            # words are a view of its storage: a slot added within its capacity keeps the address
            # and changes the slot count the descriptors carry.
            src = self._bank[0].words if self._bank is not None else self.idx_a
            key = (x.dtype, src.data_ptr(), src.shape[0], self.idx_b.data_ptr(), self.idx_b.shape[0],
                   _hip.version_of(self.pool_a), _hip.version_of(self.pool_b), slots.data_ptr(), slots.shape[0])
            if self._eager is None or self._eager[0] != key:
                self._eager = (key, self._factors(x.dtype), _delta.routes(slots))
            _, f, route = self._eager
            _delta.lora_delta(x3.contiguous(), out3, rank=self.rank, factors=f, route=route, accumulate=True,
                              out_scale=self.scaling)
            return out
        # traced: the torch.library ops (lithe_amd/kernels/ops.py), one opaque in-place op for
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
    wrapped: Dict[str, nn.Module] = {}
    for path in paths:
        linear = model.get_submodule(path)
        if not isinstance(linear, nn.Linear):
            raise TypeError(f"{path} is not nn.Linear")
        wrapped[path] = factory(path, linear)
        replace_module(model, path, wrapped[path])
    return wrapped


__all__ = ["IndexLoRALinear", "PerSampleLoRALinear", "wrap_linears", "replace_module", "per_sample_lora_delta"]
