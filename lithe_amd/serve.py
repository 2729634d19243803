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

Route = Sequence[Tuple[int, float]]  # [(adapter_id, weight), ...] for one sample


class Router:
    """Per-batch routing table shared by all MultiAdapterLinear layers."""

    def __init__(self):
        self.ids: Optional[torch.Tensor] = None      # (b, m) int64, -1 = padding
        self.weights: Optional[torch.Tensor] = None  # (b, m) float32
        self._dev: Dict[str, Tuple[torch.Tensor, torch.Tensor]] = {}

    def set(self, routes: Sequence[Route]) -> None:
        m = max(1, max((len(r) for r in routes), default=1))
        ids = torch.full((len(routes), m), -1, dtype=torch.int64)
        w = torch.zeros(len(routes), m, dtype=torch.float32)
        for i, r in enumerate(routes):
            for j, (a, wt) in enumerate(r):
                if wt < 0:
                    raise ValueError("mixture weights must be non-negative")
                ids[i, j], w[i, j] = int(a), float(wt)
        self.ids, self.weights = ids, w
        self._dev = {}

    def device_tables(self, device) -> Tuple[torch.Tensor, torch.Tensor]:
        """(slot int32 (b, m), sqrt-weight fp32 (b, m)) on ``device``, built once per ``set``.

        sqrt(max(w * valid, 0)) is evaluated in fp32 (IEEE sqrt is correctly
        rounded, as on the reference's device).
        """
        key = str(device)
        if key not in self._dev:
            ids = self.ids.numpy()
            valid = ids >= 0
            w = self.weights.numpy().astype(np.float32) * valid.astype(np.float32)
            g = np.sqrt(np.maximum(w, np.float32(0)), dtype=np.float32)
            slot = np.where(valid, ids, -1).astype(np.int32)
            self._dev[key] = (torch.from_numpy(slot).to(device), torch.from_numpy(g).to(device))
        return self._dev[key]


class MultiAdapterLinear(nn.Module):
    def __init__(self, base: nn.Linear, router: Router, rank: int, pool_a: torch.Tensor, pool_b: torch.Tensor):
        super().__init__()
        self.base = base
        self.router = router
        self.rank = rank
        self.shape_a = (rank, base.in_features)
        self.shape_b = (base.out_features, rank)
        self.register_buffer("pool_a", pool_a, persistent=False)
        self.register_buffer("pool_b", pool_b, persistent=False)
        # index banks: (n_adapters, L, n_blocks) int16 (K = 512 fits), plus per-adapter alpha / r
        self.register_buffer("idx_a", torch.zeros(0, pool_a.shape[0], quant.num_blocks(self.shape_a),
                                                  dtype=torch.int16), persistent=False)
        self.register_buffer("idx_b", torch.zeros(0, pool_b.shape[0], quant.num_blocks(self.shape_b),
                                                  dtype=torch.int16), persistent=False)
        self.register_buffer("scales", torch.zeros(0), persistent=False)

    def add_adapter(self, idx_a: np.ndarray, idx_b: np.ndarray, scale: float) -> None:
        dev = self.idx_a.device
        self.idx_a = torch.cat([self.idx_a, torch.from_numpy(np.asarray(idx_a).astype(np.int16))[None].to(dev)])
        self.idx_b = torch.cat([self.idx_b, torch.from_numpy(np.asarray(idx_b).astype(np.int16))[None].to(dev)])
        self.scales = torch.cat([self.scales, torch.tensor([scale], device=dev, dtype=torch.float32)])

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = self.base(x)
        ids = self.router.ids
        if ids is None or (ids < 0).all():
            return out
        if ids.shape[0] != x.shape[0]:
            raise ValueError(f"route batch {ids.shape[0]} != input batch {x.shape[0]}")
        n = int(self.idx_a.shape[0])
        if int(ids.max()) >= n:
            raise IndexError(f"route names adapter {int(ids.max())}, only {n} loaded")
        _hip.require_gpu(x, self.idx_a)
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
            _delta.index_source(self.idx_a, L, self.idx_a.shape[2]),
            _delta.index_source(self.idx_b, L, self.idx_b.shape[2]),
            _hip.lut_from_pools(self.pool_a, torch.float32), _hip.lut_from_pools(self.pool_b, torch.float32))
        route = _delta.routes(slot, g, self.scales.to(device=x.device, dtype=torch.float32).contiguous())
        _delta.lora_delta(xs, out3, rank=self.rank, factors=f, route=route, accumulate=True)
        return out


def attach_adapters(model: nn.Module, adapters: List[LitheAdapter],
                    router: Optional[Router] = None) -> Tuple[Router, Dict[str, MultiAdapterLinear]]:
    """Wrap every linear named in the adapters' module list and load all index streams."""
    if not adapters:
        raise ValueError("need at least one adapter")
    router = router or Router()
    ref = adapters[0]
    names = [mm["name"] for mm in ref.modules]
    for ad in adapters[1:]:
        # module sets are compared as sets: training and encode outputs may order them differently
        if {mm["name"] for mm in ad.modules} != set(names) or ad.rank != ref.rank:
            raise ValueError("all adapters must cover the same modules with the same rank")
    pool_a = cb.build_pools(ref.sigma_a, ref.block_size, ref.n_bits)
    pool_b = cb.build_pools(ref.sigma_b, ref.block_size, ref.n_bits)
    layers: Dict[str, MultiAdapterLinear] = {}
    for name in names:
        path = name[len("transformer."):] if name.startswith("transformer.") else name
        base = model.get_submodule(path)
        if not isinstance(base, nn.Linear):
            raise TypeError(f"{path} is not nn.Linear")
        parent_name, _, child = path.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        layer = MultiAdapterLinear(base, router, ref.rank, pool_a, pool_b).to(base.weight.device)
        for ad in adapters:
            layer.add_adapter(ad.indices[name]["A"], ad.indices[name]["B"], float(ad.alpha) / ad.rank)
        setattr(parent, child, layer)
        layers[name] = layer
    return router, layers


def parse_route(spec: str) -> List[Tuple[int, float]]:
    """'0' -> [(0, 1.0)];  '0:0.6,2:0.4' -> [(0, 0.6), (2, 0.4)];  'none' -> []."""
    if spec.strip().lower() in ("", "none", "-"):
        return []
    route = []
    for part in spec.split(","):
        a, _, wt = part.partition(":")
        route.append((int(a), float(wt) if wt else 1.0))
    return route
