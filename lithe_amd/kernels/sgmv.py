"""Two-stage per-sample LoRA delta over decoded factors (API of ``lithe/kernels/sgmv.py``).

For a batch in which sample ``b`` uses its own factors ``A_b`` (r, d_in) and
``B_b`` (d_out, r) with scale ``s_b``::

    delta[b, s, o] = s_b * sum_k B_b[o, k] * sum_d A_b[k, d] * x[b, s, d]

Runs through the same gfx950 shrink / expand kernels as the index-resident
path with dense factors as the source. Dtype steps follow the reference:
bf16 activations use the kernel semantics (``sgmv.py:29-100``: the scale is
applied to the fp32 ``mid`` before its bf16 rounding), fp32 activations the
bmm semantics (``sgmv.py:103-109``: the scale multiplies the delta).
"""
from __future__ import annotations

import torch

from . import _delta, _hip


def per_sample_lora_delta(x: torch.Tensor, sA: torch.Tensor, sB: torch.Tensor,
                          scaling: torch.Tensor) -> torch.Tensor:
    """Per-sample LoRA delta ``[B, seq, d_out]`` on the GPU."""
    if x.dim() != 3:
        raise ValueError(f"x must be 3D, got {tuple(x.shape)}")
    bsz, seq, in_dim = x.shape
    ba, r, in_a = sA.shape
    bb, out_dim, rb = sB.shape
    if ba != bsz or bb != bsz or scaling.shape[0] != bsz:
        raise ValueError(f"batch mismatch x={bsz} sA={ba} sB={bb} scaling={scaling.shape[0]}")
    if in_a != in_dim or r != rb:
        raise ValueError("factor shapes do not match x")
    return lora_delta_dense(x, sA, sB, scaling.to(x.dtype).float(), base=None)


def lora_delta_dense(x: torch.Tensor, sA: torch.Tensor, sB: torch.Tensor, scaling: torch.Tensor,
                     base: torch.Tensor = None, slots: torch.Tensor = None, bmm_semantics: bool = None
                     ) -> torch.Tensor:
    """Delta of per-sample dense factors; added into ``base`` in place when given.

    ``scaling`` (B,) holds the exact fp32 multipliers (callers round them the way
    the reference does). ``slots`` (B,) picks factor pair slots[b] for sample b
    (default: b). With
    ``bmm_semantics`` the scale multiplies the rounded delta (the reference's bmm
    path); otherwise it multiplies the fp32 mid before rounding (its bf16 kernel).
    """
    _hip.require_gpu(x, sA, sB, scaling)
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"lithe_amd kernels take bfloat16 or float32 activations, got {x.dtype}")
    bsz, seq, d_in = x.shape
    n, r, _ = sA.shape
    d_out = sB.shape[1]
    if d_in % 64 or (d_out * r) % 64:
        raise ValueError("d_in and d_out * r must be multiples of 64")
    a = sA.to(x.dtype).contiguous()
    b = sB.to(x.dtype).contiguous()
    if bmm_semantics is None:
        bmm_semantics = x.dtype != torch.bfloat16
    s = scaling.to(device=x.device, dtype=torch.float32).contiguous()
    if slots is None:
        slots = torch.arange(bsz, device=x.device, dtype=torch.int32)
    route = _delta.routes(slots.to(device=x.device, dtype=torch.int32).reshape(-1, 1).contiguous())
    f = _delta.dense_factors(a, b)
    if base is None:
        y = torch.empty((bsz, seq, d_out), dtype=x.dtype, device=x.device)
        acc = False
    else:
        y, acc = base, True
    if bmm_semantics:
        return _delta.lora_delta(x.contiguous(), y, rank=r, factors=f, route=route, accumulate=acc,
                                 out_scale_vec=s)
    return _delta.lora_delta(x.contiguous(), y, rank=r, factors=f, route=route, accumulate=acc, mid_scale=s)
