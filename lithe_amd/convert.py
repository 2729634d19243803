"""Conversions between index adapters and dense LoRA state dicts (``lithe/convert.py:15-118``).

``decode_factors`` decodes an adapter's index streams on the GPU, ``to_lora_state_dict``
writes the dense factors as a PEFT / Kohya state dict, and ``from_dense_lora`` encodes a
dense PEFT / diffusers LoRA into an index adapter with the GPU encode (closed-form greedy
search, ``lithe_encode``). The import of the research trainers' pickled checkpoints
(``from_training_checkpoint``) needs an unrestricted unpickler and is not part of this
library.
"""
from __future__ import annotations

import re
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from . import codebook as cb
from . import quant
from .fileio import LitheAdapter


def adapter_pools(ad: LitheAdapter) -> Tuple[torch.Tensor, torch.Tensor]:
    return (cb.build_pools(ad.sigma_a, ad.block_size, ad.n_bits),
            cb.build_pools(ad.sigma_b, ad.block_size, ad.n_bits))


def decode_factors(ad: LitheAdapter, device="cuda") -> Dict[str, Tuple[torch.Tensor, torch.Tensor]]:
    """name -> (A_hat (r, d_in), B_hat (d_out, r)), float32, decoded on the GPU."""
    pool_a, pool_b = (p.to(device) for p in adapter_pools(ad))
    out = {}
    for m in ad.modules:
        idx = ad.indices[m["name"]]
        a = quant.decode(torch.from_numpy(idx["A"].astype(np.int32)).to(device), m["shape_a"], pool_a)
        b = quant.decode(torch.from_numpy(idx["B"].astype(np.int32)).to(device), m["shape_b"], pool_b)
        out[m["name"]] = (a, b)
    return out


def to_lora_state_dict(ad: LitheAdapter, dtype: torch.dtype = torch.bfloat16,
                       device="cuda") -> Dict[str, torch.Tensor]:
    """Dense LoRA state dict (``lithe/convert.py:32-56``) on the CPU: alpha / r folded into B;
    diffusers-named adapters get PEFT keys (``transformer.<path>.lora_A.weight``), Kohya-named
    ones Kohya keys (``<name>.lora_down.weight``, ``.lora_up.weight``, ``.alpha`` = r)."""
    scale = float(ad.alpha) / ad.rank
    sd: Dict[str, torch.Tensor] = {}
    for name, (a, b) in decode_factors(ad, device).items():
        b = b * scale
        if ad.key_format == "diffusers":
            prefix = name if name.startswith("transformer.") else f"transformer.{name}"
            sd[f"{prefix}.lora_A.weight"] = a.to(dtype).cpu().contiguous()
            sd[f"{prefix}.lora_B.weight"] = b.to(dtype).cpu().contiguous()
        elif ad.key_format == "kohya":
            sd[f"{name}.lora_down.weight"] = a.to(dtype).cpu().contiguous()
            sd[f"{name}.lora_up.weight"] = b.to(dtype).cpu().contiguous()
            sd[f"{name}.alpha"] = torch.tensor(float(ad.rank), dtype=dtype)
        else:
            raise ValueError(f"unknown key_format {ad.key_format!r}")
    return sd


_PEFT_KEY = re.compile(r"^(?:base_model\.model\.)?(?:transformer\.)?(.+)\.lora_(A|B)\.weight$")


def from_dense_lora(state_dict: Dict[str, torch.Tensor], rank: Optional[int] = None,
                    base_model: str = "black-forest-labs/FLUX.1-dev", device="cuda") -> LitheAdapter:
    """Post-hoc twin-RVQ encoding of a dense PEFT / diffusers LoRA (``lithe/convert.py:61-101``):
    each ``lora_A`` / ``lora_B`` pair (alpha / r folded into B where an ``.alpha`` key is given)
    is encoded on ``device`` with the closed-form greedy search against the twin pools."""
    pairs: Dict[str, Dict[str, torch.Tensor]] = {}
    alphas: Dict[str, float] = {}
    for key, value in state_dict.items():
        m = _PEFT_KEY.match(key)
        if m:
            pairs.setdefault(m.group(1), {})[m.group(2)] = value
        elif key.endswith(".alpha"):
            alphas[re.sub(r"^(?:transformer\.)", "", key[: -len(".alpha")])] = float(value)
    if not pairs:
        raise ValueError("no PEFT-style lora_A / lora_B keys found")
    r_seen = None
    for name, ab in pairs.items():    # argument errors before any device work
        if "A" not in ab or "B" not in ab:
            raise ValueError(f"{name}: missing lora_A or lora_B")
        r = ab["A"].shape[0]
        if rank is not None and r != rank:
            raise ValueError(f"{name}: rank {r} != {rank}")
        r_seen = r
    pool_a, pool_b = (p.to(device) for p in cb.twin_pools())
    proj = cb.projection_matrix()
    modules, indices = [], {}
    for name, ab in pairs.items():
        a = ab["A"].to(device=device, dtype=torch.float32)
        b = ab["B"].to(device=device, dtype=torch.float32)
        r = a.shape[0]
        if name in alphas:
            b = b * (alphas[name] / r)
        idx_a, _ = quant.encode(a, pool_a, proj)
        idx_b, _ = quant.encode(b, pool_b, proj)
        modules.append({"name": name, "shape_a": list(a.shape), "shape_b": list(b.shape)})
        indices[name] = {"A": idx_a.cpu().numpy().astype(np.uint16), "B": idx_b.cpu().numpy().astype(np.uint16)}
    return LitheAdapter(modules=modules, indices=indices, rank=r_seen, alpha=float(r_seen), key_format="diffusers",
                        base_model=base_model,
                        metadata={"source": "post-hoc encoding of a dense LoRA", "module_set": f"diffusers-{len(modules)}"})
