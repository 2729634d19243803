"""``torch.library`` operators over the C ABI, so that ``torch.compile`` / FX trace the layers
with the delta as one opaque op that mutates the base output in place.

* ``lithe_amd::bank_lora_delta_(x, y, words, a_off, b_off, pool_a, pool_b, slots, rank, scaling)``:
  y += delta of the module whose A / B blocks start at ``a_off`` / ``b_off`` of the packed bank
  ``words`` (n_slots, n_words); sample i uses slot ``slots[i, 0]``.
* ``lithe_amd::index_lora_delta_(x, y, idx_a, idx_b, pool_a, pool_b, slots, rank, scaling)``:
  the same over level-major int16 or int32 index stacks (n_slots, L, n_blocks) -- ``IndexLoRALinear``
  built from tensors (``lithe/kernels/layers.py:97-131``).

Both run ``lithe_lora_delta`` with the rounding of ``out + delta * scaling``
(``lithe/kernels/shared.py:261-262``, ``layers.py:131``) on the current stream. Their fake
implementations return nothing: the only effect is the in-place update of ``y``.
"""
from __future__ import annotations

import torch

from . import _delta, _hip


def _run(x: torch.Tensor, y: torch.Tensor, a_src, b_src, pool_a: torch.Tensor, pool_b: torch.Tensor,
         slots: torch.Tensor, rank: int, scaling: float) -> None:
    f = _delta.indexed_factors(a_src, b_src, _hip.lut_from_pools(pool_a, x.dtype), _hip.lut_from_pools(pool_b, x.dtype))
    _delta.lora_delta(x, y, rank=rank, factors=f, route=_delta.routes(slots), accumulate=True, out_scale=scaling)


@torch.library.custom_op("lithe_amd::bank_lora_delta_", mutates_args=("y",), device_types="cuda")
def bank_lora_delta_(x: torch.Tensor, y: torch.Tensor, words: torch.Tensor, a_off: int, b_off: int,
                     pool_a: torch.Tensor, pool_b: torch.Tensor, slots: torch.Tensor, rank: int,
                     scaling: float) -> None:
    L = int(pool_a.shape[0])
    _run(x, y, _delta.packed_source(words, L, a_off), _delta.packed_source(words, L, b_off), pool_a, pool_b, slots,
         rank, scaling)


@bank_lora_delta_.register_fake
def _bank_lora_delta_fake(x, y, words, a_off, b_off, pool_a, pool_b, slots, rank, scaling) -> None:
    return None


@torch.library.custom_op("lithe_amd::index_lora_delta_", mutates_args=("y",), device_types="cuda")
def index_lora_delta_(x: torch.Tensor, y: torch.Tensor, idx_a: torch.Tensor, idx_b: torch.Tensor,
                      pool_a: torch.Tensor, pool_b: torch.Tensor, slots: torch.Tensor, rank: int,
                      scaling: float) -> None:
    L = int(pool_a.shape[0])
    d_in, d_out = x.shape[-1], y.shape[-1]
    _run(x, y, _delta.index_source(idx_a, L, rank * d_in // 64), _delta.index_source(idx_b, L, d_out * rank // 64),
         pool_a, pool_b, slots, rank, scaling)


@index_lora_delta_.register_fake
def _index_lora_delta_fake(x, y, idx_a, idx_b, pool_a, pool_b, slots, rank, scaling) -> None:
    return None
