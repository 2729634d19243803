"""LITHE LoRA linear wrapper and injection (inference half of ``lithe/module.py``).

``LitheLinear.load_indices`` decodes the index streams to fp32 factors once on
the GPU (``quant.decode``, bit-identical to the reference's fp32 decode);
``forward`` adds ``(x A^T) B^T * alpha / r`` to the base output through the
gfx950 shrink / expand kernels with the reference's rounding steps
(``module.py:145-156``: each product rounded to the activation dtype, then
``delta * scaling``, then ``out + delta``). Training (STE re-quantisation,
``module.py:240-264``) is not part of this library.
"""
from __future__ import annotations

import math
from typing import Dict, Iterable, List, Optional, Sequence

import torch
from torch import nn

from . import codebook as cb
from . import quant

# FLUX.1-dev (diffusers FluxTransformer2DModel) attention + FFN linears.
# Suffix match over module paths gives 19 x 12 + 38 x 3 = 342 linears.
FLUX_TARGET_MODULES: List[str] = [
    "attn.to_q",
    "attn.to_k",
    "attn.to_v",
    "attn.to_out.0",
    "attn.add_q_proj",
    "attn.add_k_proj",
    "attn.add_v_proj",
    "attn.to_add_out",
    "ff.net.0.proj",
    "ff.net.2",
    "ff_context.net.0.proj",
    "ff_context.net.2",
]


class TwinCodebook(nn.Module):
    """Holds the deterministic pools as non-persistent buffers (never saved)."""

    def __init__(self, block_size: int = cb.BLOCK_SIZE, n_bits: int = cb.N_BITS,
                 sigma_a: Sequence[float] = cb.SIGMA_A, sigma_b: Sequence[float] = cb.SIGMA_B):
        super().__init__()
        pool_a, pool_b = cb.twin_pools(block_size, n_bits, sigma_a, sigma_b)
        self.block_size = block_size
        self.n_bits = n_bits
        self.sigma_a = tuple(float(s) for s in sigma_a)
        self.sigma_b = tuple(float(s) for s in sigma_b)
        self.register_buffer("pool_a", pool_a, persistent=False)
        self.register_buffer("pool_b", pool_b, persistent=False)
        self.register_buffer("proj", cb.projection_matrix(block_size, n_bits), persistent=False)
        self._per_device: Dict[str, tuple] = {}

    def tensors(self, device) -> tuple:
        """(pool_a, pool_b, proj) on ``device``; copied once per device."""
        key = str(device)
        if key not in self._per_device:
            self._per_device[key] = (self.pool_a.to(device), self.pool_b.to(device), self.proj.to(device))
        return self._per_device[key]

    def encode(self, w: torch.Tensor, side: str):
        raise NotImplementedError("encoding (the training-time search) is not part of lithe_amd")

    def decode(self, indices: torch.Tensor, shape, side: str) -> torch.Tensor:
        pool_a, pool_b, _ = self.tensors(indices.device)
        return quant.decode(indices, shape, pool_a if side == "A" else pool_b)


class LitheLinear(nn.Module):
    """y = W x + (B_hat A_hat x) * alpha / r with A_hat, B_hat decoded from index streams."""

    def __init__(self, base: nn.Linear, codebook: TwinCodebook, rank: int = 16,
                 alpha: Optional[float] = None, requantize_every: int = 10,
                 drift_tau: Optional[float] = None):
        super().__init__()
        self.base = base
        for p in self.base.parameters():
            p.requires_grad_(False)
        self.in_features = base.in_features
        self.out_features = base.out_features
        self.rank = rank
        self.alpha = float(rank if alpha is None else alpha)
        self.scaling = self.alpha / rank
        self.requantize_every = max(1, int(requantize_every))
        self.drift_tau = drift_tau
        # Not registered as a submodule: one codebook is shared by all wrappers.
        self.__dict__["codebook"] = codebook
        device = base.weight.device
        self.lora_A = nn.Parameter(torch.empty(rank, self.in_features, device=device, dtype=torch.float32))
        self.lora_B = nn.Parameter(torch.zeros(self.out_features, rank, device=device, dtype=torch.float32))
        nn.init.kaiming_uniform_(self.lora_A, a=math.sqrt(5))
        self._cache_A: Optional[torch.Tensor] = None
        self._cache_B: Optional[torch.Tensor] = None
        self._frozen = False

    @torch.no_grad()
    def load_indices(self, idx_a: torch.Tensor, idx_b: torch.Tensor) -> None:
        """Freeze the module to the factors decoded from index streams (fp32, on the GPU)."""
        dev = self.lora_A.device
        self._cache_A = self.codebook.decode(idx_a.to(dev), self.lora_A.shape, "A")
        self._cache_B = self.codebook.decode(idx_b.to(dev), self.lora_B.shape, "B")
        self._frozen = True
        self.lora_A.requires_grad_(False)
        self.lora_B.requires_grad_(False)

    def decoded_factors(self):
        """(A_hat, B_hat) float32 as used by the forward pass."""
        if self._cache_A is None:
            raise NotImplementedError("no indices loaded: re-quantising the fp32 proxies is training, "
                                      "which is not part of lithe_amd; call load_indices first")
        return self._cache_A, self._cache_B

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not (self._frozen or not self.training):
            raise NotImplementedError("LitheLinear training (STE) is not part of lithe_amd; call load_indices")
        from .kernels.sgmv import lora_delta_dense
        out = self.base(x)
        a_hat, b_hat = self.decoded_factors()
        x3 = x.reshape(1, -1, x.shape[-1])
        if not out.is_contiguous():
            out = out.contiguous()
        out3 = out.view(1, -1, out.shape[-1])
        scale = torch.full((1,), self.scaling, dtype=torch.float32, device=x.device)
        lora_delta_dense(x3, a_hat.unsqueeze(0), b_hat.unsqueeze(0), scale, base=out3,
                         slots=torch.zeros(1, dtype=torch.int32, device=x.device), bmm_semantics=True)
        return out


def _match(path: str, targets: Iterable[str]) -> bool:
    return any(path == t or path.endswith("." + t) for t in targets)


def inject_lithe(model: nn.Module, target_modules: Sequence[str] = FLUX_TARGET_MODULES,
                 rank: int = 16, alpha: Optional[float] = None, requantize_every: int = 10,
                 drift_tau: Optional[float] = None,
                 codebook: Optional[TwinCodebook] = None) -> Dict[str, LitheLinear]:
    """Replace every nn.Linear whose path ends with a target suffix by a LitheLinear.

    Returns an ordered {module_path: LitheLinear}; this order defines the layout
    of the index stream.
    """
    codebook = codebook if codebook is not None else TwinCodebook()
    targets = [(name, mod) for name, mod in model.named_modules()
               if isinstance(mod, nn.Linear) and _match(name, target_modules)]
    if not targets:
        raise ValueError("no target linear found; check target_modules")
    wrapped: Dict[str, LitheLinear] = {}
    for name, mod in targets:
        parent_name, _, child = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        layer = LitheLinear(mod, codebook, rank=rank, alpha=alpha, requantize_every=requantize_every,
                            drift_tau=drift_tau)
        setattr(parent, child, layer)
        wrapped[name] = layer
    return wrapped


def lithe_layers(model: nn.Module) -> Dict[str, LitheLinear]:
    return {n: m for n, m in model.named_modules() if isinstance(m, LitheLinear)}
