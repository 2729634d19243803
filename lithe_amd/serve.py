"""Index-resident multi-adapter serving: heterogeneous adapters in one forward.

API of ``lithe/serve.py``. Every wrapped linear keeps only the int16 index
streams of all loaded adapters. For each forward, sample i gets the
rank-stacked update

    A_i = vcat_a[ sqrt(w_ia) A_a ],  B_i = hcat_a[ sqrt(w_ia) s_a B_a ],  delta_i = B_i A_i x_i

(one adapter, a weighted mixture, or none). The reference decodes the active
adapters densely and runs two bmm (``serve.py:69-97``); here one
``lithe_lora_delta`` call decodes the factors inside the gfx950 shrink / expand
tiles, with the same dtype steps: fp32 decode from fp32 pools, ``alpha / r``
and sqrt(w) multiplied in fp32, factors cast to the activation dtype,
``x A^T`` rounded to the activation dtype, ``(x A^T) B^T`` rounded, then
``out + delta``. Up to 8 route entries per sample at rank 16.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch
from torch import nn

from . import codebook as cb
from . import quant
from .fileio import LitheAdapter
from .kernels import _delta, _hip
from .kernels.layers import replace_module

Route = Sequence[Tuple[int, float]]  # [(adapter_id, weight), ...] for one sample


class Router:
    """Routing table of the current batch, shared by every ``MultiAdapterLinear`` of a model
    (``lithe/serve.py:28-44``).

    ``ids`` is (batch, width) int64 with -1 in unused entries and ``weights`` the matching
    fp32 mixture weights; width is the longest route (at least 1). The kernels read the
    int32 slot table and the fp32 square roots of the weights, built once per device per ``set``.
    """

    def __init__(self):
        self.ids: Optional[torch.Tensor] = None
        self.weights: Optional[torch.Tensor] = None
        self._device_tables: Dict[str, Tuple[torch.Tensor, torch.Tensor]] = {}

    def set(self, routes: Sequence[Route]) -> None:
        entries = [[(int(a), float(w)) for a, w in r] for r in routes]
        if any(w < 0 for r in entries for _, w in r):
            raise ValueError("mixture weights must be non-negative")
        width = max([len(r) for r in entries] + [1])
        ids = np.full((len(entries), width), -1, dtype=np.int64)
        wts = np.zeros((len(entries), width), dtype=np.float32)
        for row, r in enumerate(entries):
            if r:
                ids[row, :len(r)], wts[row, :len(r)] = zip(*r)
        self.ids, self.weights = torch.from_numpy(ids), torch.from_numpy(wts)
        self._device_tables = {}

    def device_tables(self, device) -> Tuple[torch.Tensor, torch.Tensor]:
        """(slot int32 (b, m), sqrt-weight fp32 (b, m)) on ``device``, built once per ``set``.

        sqrt(max(w * valid, 0)) is evaluated in fp32 (IEEE sqrt is correctly
        rounded, as on the reference's device).
        """
        key = str(device)
        if key not in self._device_tables:
            ids = self.ids.numpy()
            used = ids >= 0
            root = np.sqrt(np.maximum(self.weights.numpy() * used, np.float32(0)), dtype=np.float32)
            slots = np.where(used, ids, -1).astype(np.int32)
            self._device_tables[key] = (torch.from_numpy(slots).to(device), torch.from_numpy(root).to(device))
        return self._device_tables[key]


class MultiAdapterLinear(nn.Module):
    """``base(x)`` plus each sample's routed adapter deltas, decoded from resident int16 indices.

    ``idx_a`` / ``idx_b`` ((n_adapters, L, n_blocks) int16) and ``scales`` ((n_adapters,) fp32
    alpha / r) are views of stores that double their capacity as adapters are added, so loading
    n adapters copies O(n) index rows, not O(n^2).
    """

    def __init__(self, base: nn.Linear, router: Router, rank: int, pool_a: torch.Tensor, pool_b: torch.Tensor):
        super().__init__()
        self.base = base
        self.router = router
        self.rank = rank
        self.shape_a = (rank, base.in_features)
        self.shape_b = (base.out_features, rank)
        self.register_buffer("pool_a", pool_a, persistent=False)
        self.register_buffer("pool_b", pool_b, persistent=False)
        self._n = 0
        self._alloc(1)

    def _alloc(self, capacity: int) -> None:
        """(Re)allocate the stores for ``capacity`` adapters, keeping the loaded ones."""
        dev = self.pool_a.device
        grown = {
            "_store_a": torch.zeros((capacity, self.pool_a.shape[0], quant.num_blocks(self.shape_a)),
                                    dtype=torch.int16, device=dev),
            "_store_b": torch.zeros((capacity, self.pool_b.shape[0], quant.num_blocks(self.shape_b)),
                                    dtype=torch.int16, device=dev),
            "_store_s": torch.zeros(capacity, dtype=torch.float32, device=dev),
        }
        for name, t in grown.items():
            if self._n:
                t[: self._n].copy_(getattr(self, name)[: self._n])
            self.register_buffer(name, t, persistent=False)

    @property
    def idx_a(self) -> torch.Tensor:
        return self._store_a[: self._n]

    @property
    def idx_b(self) -> torch.Tensor:
        return self._store_b[: self._n]

    @property
    def scales(self) -> torch.Tensor:
        return self._store_s[: self._n]

    def add_adapter(self, idx_a: np.ndarray, idx_b: np.ndarray, scale: float) -> None:
        a = torch.from_numpy(np.ascontiguousarray(np.asarray(idx_a).astype(np.int16)))
        b = torch.from_numpy(np.ascontiguousarray(np.asarray(idx_b).astype(np.int16)))
        if a.shape != self._store_a.shape[1:] or b.shape != self._store_b.shape[1:]:
            raise ValueError(f"adapter indices {tuple(a.shape)} / {tuple(b.shape)} do not fit the layer "
                             f"({tuple(self._store_a.shape[1:])} / {tuple(self._store_b.shape[1:])})")
        if self._n == self._store_a.shape[0]:
            self._alloc(2 * self._n)
        self._store_a[self._n].copy_(a)
        self._store_b[self._n].copy_(b)
        self._store_s[self._n] = float(scale)
        self._n += 1

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = self.base(x)
        ids = self.router.ids
        if ids is None or (ids < 0).all():
            return out
        if ids.shape[0] != x.shape[0]:
            raise ValueError(f"route batch {ids.shape[0]} != input batch {x.shape[0]}")
        n = self._n
        if int(ids.max()) >= n:
            raise IndexError(f"route names adapter {int(ids.max())}, only {n} loaded")
        _hip.require_gpu(x, self._store_a)
        if x.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError(f"lithe_amd kernels take bfloat16 or float32 activations, got {x.dtype}")
        if -(-self.rank // 16) * ids.shape[1] > 8:
            raise ValueError("at most 8 groups of 16 ranks per sample (route length x ceil(rank / 16))")
        slot, g = self.router.device_tables(x.device)
        bsz = ids.shape[0]
        xs = x.reshape(bsz, -1, x.shape[-1]).contiguous()
        if not out.is_contiguous():
            out = out.contiguous()
        out3 = out.view(bsz, -1, out.shape[-1])
        L = int(self.pool_a.shape[0])
        f = _delta.indexed_factors(
            _delta.index_source(self.idx_a, L, self._store_a.shape[2]),
            _delta.index_source(self.idx_b, L, self._store_b.shape[2]),
            _hip.lut_from_pools(self.pool_a, torch.float32), _hip.lut_from_pools(self.pool_b, torch.float32))
        route = _delta.routes(slot, g, self._store_s)
        _delta.lora_delta(xs, out3, rank=self.rank, factors=f, route=route, accumulate=True)
        return out


def _target_path(name: str) -> str:
    """Module path inside the transformer of an adapter's module name (an optional
    ``transformer.`` prefix names the same module)."""
    prefix = "transformer."
    return name[len(prefix):] if name.startswith(prefix) else name


def attach_adapters(model: nn.Module, adapters: List[LitheAdapter],
                    router: Optional[Router] = None) -> Tuple[Router, Dict[str, MultiAdapterLinear]]:
    """Replace every linear the adapters name by a ``MultiAdapterLinear`` holding all of their
    index streams (adapter i = route id i); returns the shared router and the layers by name."""
    if not adapters:
        raise ValueError("need at least one adapter")
    first = adapters[0]
    names = [entry["name"] for entry in first.modules]
    # adapters may list their modules in different orders (training vs encode output)
    if any({e["name"] for e in ad.modules} != set(names) or ad.rank != first.rank for ad in adapters):
        raise ValueError("all adapters must cover the same modules with the same rank")
    router = router if router is not None else Router()
    pools = (cb.build_pools(first.sigma_a, first.block_size, first.n_bits),
             cb.build_pools(first.sigma_b, first.block_size, first.n_bits))
    scales = [float(ad.alpha) / ad.rank for ad in adapters]
    layers: Dict[str, MultiAdapterLinear] = {}
    for name in names:
        path = _target_path(name)
        linear = model.get_submodule(path)
        if not isinstance(linear, nn.Linear):
            raise TypeError(f"{path} is not nn.Linear")
        wrapped = MultiAdapterLinear(linear, router, first.rank, *pools).to(linear.weight.device)
        for ad, s in zip(adapters, scales):
            wrapped.add_adapter(ad.indices[name]["A"], ad.indices[name]["B"], s)
        replace_module(model, path, wrapped)
        layers[name] = wrapped
    return router, layers


def parse_route(spec: str) -> List[Tuple[int, float]]:
    """'0' -> [(0, 1.0)];  '0:0.6,2:0.4' -> [(0, 0.6), (2, 0.4)];  'none' -> []."""
    text = spec.strip()
    if text.lower() in ("", "none", "-"):
        return []
    route = []
    for item in text.split(","):
        adapter, has_weight, weight = item.strip().partition(":")
        route.append((int(adapter), float(weight) if has_weight and weight.strip() else 1.0))
    return route
