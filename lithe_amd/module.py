"""LITHE LoRA linear wrapper and injection (inference half of ``lithe/module.py``).

``LitheLinear.load_indices`` decodes the index streams to fp32 factors once on
the GPU (``quant.decode``, bit-identical to the reference's fp32 decode);
``forward`` adds ``(x A^T) B^T * alpha / r`` to the base output through the
gfx950 shrink / expand kernels with the reference's rounding steps
(``module.py:145-156``: each product rounded to the activation dtype, then
``delta * scaling``, then ``out + delta``). Training (STE re-quantisation,
``module.py:240-264``) is not part of this library; ``TwinCodebook.encode`` is the
GPU re-quantisation of a factor (``quant.encode``).
"""
from __future__ import annotations

from typing import Dict, Iterable, List, Optional, Sequence, Tuple

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
    """The two pool stacks of one codebook configuration and its Hadamard generator, as
    non-persistent buffers (they are a function of the configuration and never saved)
    (``lithe/module.py:31-60``). Side "A" selects ``pool_a``, any other side ``pool_b``."""

    def __init__(self, block_size: int = cb.BLOCK_SIZE, n_bits: int = cb.N_BITS,
                 sigma_a: Sequence[float] = cb.SIGMA_A, sigma_b: Sequence[float] = cb.SIGMA_B):
        super().__init__()
        self.block_size, self.n_bits = block_size, n_bits
        self.sigma_a = tuple(map(float, sigma_a))
        self.sigma_b = tuple(map(float, sigma_b))
        pools = cb.twin_pools(block_size, n_bits, self.sigma_a, self.sigma_b)
        for name, t in zip(("pool_a", "pool_b", "proj"), (*pools, cb.projection_matrix(block_size, n_bits))):
            self.register_buffer(name, t, persistent=False)
        self._copies: Dict[str, Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = {}

    def tensors(self, device) -> tuple:
        """(pool_a, pool_b, proj) on ``device``; copied once per device."""
        key = str(device)
        got = self._copies.get(key)
        if got is None:
            got = self._copies[key] = tuple(t.to(device) for t in (self.pool_a, self.pool_b, self.proj))
        return got

    def _pool(self, side: str, device) -> torch.Tensor:
        pool_a, pool_b, _ = self.tensors(device)
        return pool_a if side == "A" else pool_b

    def encode(self, w: torch.Tensor, side: str):
        """(indices (L, n_blocks) int64, w_hat with w's shape) of a GPU factor: the greedy
        residual encode against this side's pools (``quant.encode``)."""
        return quant.encode(w, self._pool(side, w.device), self.tensors(w.device)[2])

    def decode(self, indices: torch.Tensor, shape, side: str) -> torch.Tensor:
        return quant.decode(indices, shape, self._pool(side, indices.device))


class LitheLinear(nn.Module):
    """y = W x + (B_hat A_hat x) * alpha / r with A_hat, B_hat decoded from index streams.

    Keeps the reference's attributes (``lora_A`` (r, d_in) and ``lora_B`` (d_out, r) fp32
    parameters, ``scaling = alpha / r``, the shared ``codebook``); the proxies only fix the
    factor shapes and device here (inference needs no initialisation of them).
    """

    def __init__(self, base: nn.Linear, codebook: TwinCodebook, rank: int = 16,
                 alpha: Optional[float] = None, requantize_every: int = 10,
                 drift_tau: Optional[float] = None):
        super().__init__()
        base.requires_grad_(False)
        self.base = base
        self.in_features, self.out_features = base.in_features, base.out_features
        self.rank = rank
        self.alpha = float(rank) if alpha is None else float(alpha)
        self.scaling = self.alpha / rank
        self.requantize_every = max(1, int(requantize_every))
        self.drift_tau = drift_tau
        object.__setattr__(self, "codebook", codebook)     # shared by every wrapper: not a submodule
        dev = base.weight.device
        self.lora_A = nn.Parameter(torch.zeros(rank, self.in_features, device=dev), requires_grad=False)
        self.lora_B = nn.Parameter(torch.zeros(self.out_features, rank, device=dev), requires_grad=False)
        self._cache_A: Optional[torch.Tensor] = None
        self._cache_B: Optional[torch.Tensor] = None
        self._frozen = False

    @torch.no_grad()
    def load_indices(self, idx_a: torch.Tensor, idx_b: torch.Tensor) -> None:
        """Freeze the module to the factors decoded from index streams (fp32, on the GPU)."""
        dev = self.lora_A.device
        self._cache_A = self.codebook.decode(idx_a.to(dev), tuple(self.lora_A.shape), "A")
        self._cache_B = self.codebook.decode(idx_b.to(dev), tuple(self.lora_B.shape), "B")
        self._frozen = True

    def decoded_factors(self):
        """(A_hat, B_hat) float32 as used by the forward pass."""
        if self._cache_A is None:
            raise NotImplementedError("no indices loaded: re-quantising the fp32 proxies is training, "
                                      "which is not part of lithe_amd; call load_indices first")
        return self._cache_A, self._cache_B

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.training and not self._frozen:
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
    """True when ``path`` is a target or ends with ``.`` + a target (whole path components)."""
    parts = path.split(".")
    return any(parts[len(parts) - len(t.split(".")):] == t.split(".") for t in targets)


def inject_lithe(model: nn.Module, target_modules: Sequence[str] = FLUX_TARGET_MODULES,
                 rank: int = 16, alpha: Optional[float] = None, requantize_every: int = 10,
                 drift_tau: Optional[float] = None,
                 codebook: Optional[TwinCodebook] = None) -> Dict[str, LitheLinear]:
    """Replace every nn.Linear whose path ends with a target suffix by a LitheLinear.

    Returns an ordered {module_path: LitheLinear}; this order defines the layout
    of the index stream.
    """
    book = TwinCodebook() if codebook is None else codebook
    found = [path for path, m in model.named_modules() if isinstance(m, nn.Linear) and _match(path, target_modules)]
    if not found:
        raise ValueError("no target linear found; check target_modules")
    from .kernels.layers import replace_module
    wrapped: Dict[str, LitheLinear] = {}
    for path in found:
        wrapped[path] = LitheLinear(model.get_submodule(path), book, rank=rank, alpha=alpha,
                                    requantize_every=requantize_every, drift_tau=drift_tau)
        replace_module(model, path, wrapped[path])
    return wrapped


def lithe_layers(model: nn.Module) -> Dict[str, LitheLinear]:
    """Every LitheLinear of ``model`` by module path."""
    return {path: m for path, m in model.named_modules() if isinstance(m, LitheLinear)}
