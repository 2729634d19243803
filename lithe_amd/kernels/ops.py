"""``torch.library`` operators over the C ABI, so that ``torch.compile`` / FX trace the layers
with the delta as one opaque op that mutates the base output in place.

* ``lithe_amd::bank_lora_delta_(x, y, words, a_off, b_off, pool_a, pool_b, slots, rank, scaling)``:
  y += delta of the module whose A / B blocks start at ``a_off`` / ``b_off`` of the packed bank
  ``words`` (n_slots, n_words); sample i uses slot ``slots[i, 0]``.
* ``lithe_amd::index_lora_delta_(x, y, idx_a, idx_b, pool_a, pool_b, slots, rank, scaling)``:
  the same over level-major int16 or int32 index stacks (n_slots, L, n_blocks) -- ``IndexLoRALinear``
  built from tensors (``lithe/kernels/layers.py:97-131``).

* ``lithe_amd::bank_lora_delta_grouped_(xs, ys, words, a_offs, b_offs, pool_a, pool_b, slots, rank, scales)``:
  the modules of one block stage in one grouped call (``lithe_lora_delta_grouped``).

All run ``lithe_lora_delta`` (the grouped op ``lithe_lora_delta_grouped``) with the rounding of ``out + delta * scaling``
(``lithe/kernels/shared.py:261-262``, ``layers.py:131``) on the current stream. Their fake
implementations return nothing: the only effect is the in-place update of ``y``.
"""
from __future__ import annotations

from typing import List

import torch

from . import _delta, _hip


def _run(x: torch.Tensor, y: torch.Tensor, a_src, b_src, pool_a: torch.Tensor, pool_b: torch.Tensor,
         slots: torch.Tensor, rank: int, scaling: float) -> None:
    f = _delta.indexed_factors(a_src, b_src, _hip.lut_from_pools(pool_a, x.dtype), _hip.lut_from_pools(pool_b, x.dtype))
    _delta.lora_delta(x, y, rank=rank, factors=f, route=_delta.routes(slots), accumulate=True, out_scale=scaling)


def bank_delta(x: torch.Tensor, y: torch.Tensor, words: torch.Tensor, a_off: int, b_off: int,
               pool_a: torch.Tensor, pool_b: torch.Tensor, slots: torch.Tensor, rank: int, scaling: float) -> None:
    """The body of ``lithe_amd::bank_lora_delta_``, called directly in eager mode."""
    L = int(pool_a.shape[0])
    _run(x, y, _delta.packed_source(words, L, a_off), _delta.packed_source(words, L, b_off), pool_a, pool_b, slots,
         rank, scaling)


def index_delta(x: torch.Tensor, y: torch.Tensor, idx_a: torch.Tensor, idx_b: torch.Tensor,
                pool_a: torch.Tensor, pool_b: torch.Tensor, slots: torch.Tensor, rank: int, scaling: float) -> None:
    """The body of ``lithe_amd::index_lora_delta_``, called directly in eager mode."""
    L = int(pool_a.shape[0])
    d_in, d_out = x.shape[-1], y.shape[-1]
    _run(x, y, _delta.index_source(idx_a, L, rank * d_in // 64), _delta.index_source(idx_b, L, d_out * rank // 64),
         pool_a, pool_b, slots, rank, scaling)


@torch.library.custom_op("lithe_amd::bank_lora_delta_", mutates_args=("y",), device_types="cuda")
def bank_lora_delta_(x: torch.Tensor, y: torch.Tensor, words: torch.Tensor, a_off: int, b_off: int,
                     pool_a: torch.Tensor, pool_b: torch.Tensor, slots: torch.Tensor, rank: int,
                     scaling: float) -> None:
    bank_delta(x, y, words, a_off, b_off, pool_a, pool_b, slots, rank, scaling)


@bank_lora_delta_.register_fake
def _bank_lora_delta_fake(x, y, words, a_off, b_off, pool_a, pool_b, slots, rank, scaling) -> None:
    return None


@torch.library.custom_op("lithe_amd::index_lora_delta_", mutates_args=("y",), device_types="cuda")
def index_lora_delta_(x: torch.Tensor, y: torch.Tensor, idx_a: torch.Tensor, idx_b: torch.Tensor,
                      pool_a: torch.Tensor, pool_b: torch.Tensor, slots: torch.Tensor, rank: int,
                      scaling: float) -> None:
    index_delta(x, y, idx_a, idx_b, pool_a, pool_b, slots, rank, scaling)


@index_lora_delta_.register_fake
def _index_lora_delta_fake(x, y, idx_a, idx_b, pool_a, pool_b, slots, rank, scaling) -> None:
    return None


def bank_delta_grouped(xs: List[torch.Tensor], ys: List[torch.Tensor], words: torch.Tensor, a_offs: List[int],
                       b_offs: List[int], pool_a: torch.Tensor, pool_b: torch.Tensor, slots: torch.Tensor,
                       rank: int, scales: List[float]) -> None:
    """ys[m] += delta of module m (blocks at a_offs[m] / b_offs[m] of the packed bank) over xs[m],
    every module in one shrink and one expand launch (``lithe_lora_delta_grouped``); modules
    given the same x tensor share its shrink. The body of ``lithe_amd::bank_lora_delta_grouped_``,
    called directly in eager mode."""
    import ctypes
    from .prepared import group_workspace_bytes
    n = len(xs)
    L = int(pool_a.shape[0])
    f = _delta.indexed_factors(_delta.packed_source(words, L, 0), _delta.packed_source(words, L, 0),
                               _hip.lut_from_pools(pool_a, xs[0].dtype), _hip.lut_from_pools(pool_b, xs[0].dtype))
    mods = (_hip.Module * n)()
    keys = {}
    for i, (x, y) in enumerate(zip(xs, ys)):
        mods[i].x, mods[i].y = x.data_ptr(), y.data_ptr()
        mods[i].seq, mods[i].d_in, mods[i].d_out = x.shape[1], x.shape[2], y.shape[2]
        mods[i].a_block_off, mods[i].b_block_off, mods[i].out_scale = int(a_offs[i]), int(b_offs[i]), float(scales[i])
        keys.setdefault(x.data_ptr(), len(keys))
    bsz = xs[0].shape[0]
    need = group_workspace_bytes([(x.shape[1], x.shape[2], y.shape[2]) for x, y in zip(xs, ys)],
                                 [keys[x.data_ptr()] for x in xs], bsz, rank, 1, xs[0].dtype)
    ws = _hip.workspace(xs[0].device, need)
    route = _delta.routes(slots)
    rc = _hip.load().lithe_lora_delta_grouped(n, mods, _hip.dtype_code(xs[0].dtype), _hip.dtype_code(ys[0].dtype), bsz,
                                              1, rank, ctypes.byref(f), ctypes.byref(route), _hip.ptr(ws), ws.numel(),
                                              _hip.stream_of(xs[0].device))
    _hip.check(rc, "lithe_lora_delta_grouped")


@torch.library.custom_op("lithe_amd::bank_lora_delta_grouped_", mutates_args=("ys",), device_types="cuda")
def bank_lora_delta_grouped_(xs: List[torch.Tensor], ys: List[torch.Tensor], words: torch.Tensor, a_offs: List[int],
                             b_offs: List[int], pool_a: torch.Tensor, pool_b: torch.Tensor, slots: torch.Tensor,
                             rank: int, scales: List[float]) -> None:
    bank_delta_grouped(xs, ys, words, a_offs, b_offs, pool_a, pool_b, slots, rank, scales)


@bank_lora_delta_grouped_.register_fake
def _bank_lora_delta_grouped_fake(xs, ys, words, a_offs, b_offs, pool_a, pool_b, slots, rank, scales) -> None:
    return None
