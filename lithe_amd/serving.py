"""Wrapping a transformer's linears for multi-adapter serving (``serving/_common.py:276-311``).

* ``select_paths`` / ``wrap_index`` / ``set_assign`` keep the reference's names and
  semantics: every target linear becomes an ``IndexLoRALinear`` holding the index slots of
  all adapters as per-layer int32 stacks, and ``set_assign`` routes the samples.
* ``wrap_bank`` is the resident-bank form: every target linear reads its slots straight
  from one ``PackedBank`` (no per-layer copies; a cold swap into the bank is visible to
  every layer at once). With ``fuse_shared_inputs`` the projections that read one input
  (``to_q`` / ``to_k`` / ``to_v``, ``add_q_proj`` / ``add_k_proj`` / ``add_v_proj``) share
  one shrink over x in one grouped call (``lithe_lora_delta_grouped``).
* ``wrap_bank(group_attention=True)`` puts the six q / k / v projections of each FLUX
  double-block attention into one grouped call made when the attention module is entered
  (``AttentionGroup``: a forward pre-hook reads ``hidden_states`` and ``encoder_hidden_states``).
* ``stage_groups`` collects the independent linears of each FLUX block stage (image and text
  projections, the two attention outputs, the two up and the two down projections) into
  ``StageGroup`` objects that add all of a stage's deltas in one grouped call
  (``lithe_lora_delta_grouped``), for a serving step that issues a stage at once.
* ``wrap_decoded`` / ``install_per_sample`` / ``install_single`` are the decoded-mode
  counterparts (``serving/_common.py:268-281``), and ``install_decoded_bank`` installs the
  stacked factors of ``PackedBank.decode_stacked`` without per-module copies.

Model loading and rendering (diffusers pipelines) are not part of this package.
"""
from __future__ import annotations

import weakref
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch
from torch import nn

from .kernels import _hip
from .kernels import ops as _ops
from .kernels.bank import PackedBank
from .kernels.layers import IndexLoRALinear, PerSampleLoRALinear, replace_module, wrap_linears
from .module import FLUX_TARGET_MODULES
from . import codebook as cb

SHARED_INPUT_GROUPS = (("attn.to_q", "attn.to_k", "attn.to_v"),
                       ("attn.add_q_proj", "attn.add_k_proj", "attn.add_v_proj"))


def _grouped_delta(xs, ys, words, a_offs, b_offs, pool_a, pool_b, slots, rank, scales) -> None:
    """One grouped delta call: the torch.library op when traced (torch.compile), its body directly
    in eager mode (no dispatcher on the host path)."""
    if torch.compiler.is_compiling():
        torch.ops.lithe_amd.bank_lora_delta_grouped_(xs, ys, words, a_offs, b_offs, pool_a, pool_b, slots, rank,
                                                     scales)
    else:
        _ops.bank_delta_grouped(xs, ys, words, a_offs, b_offs, pool_a, pool_b, slots, rank, scales)


def select_paths(paths: Sequence[str], module_set: str = "all") -> List[str]:
    """``all``: every path; ``attn-ff``: the attention / feed-forward linears of
    ``FLUX_TARGET_MODULES`` (``serving/_common.py:284-291``)."""
    if module_set == "all":
        return list(paths)
    if module_set == "attn-ff":
        return [p for p in paths if any(p.endswith(s) for s in FLUX_TARGET_MODULES)]
    raise ValueError(f"unknown module set {module_set!r}")


def wrap_index(model: nn.Module, ads, device, dtype: torch.dtype = torch.bfloat16,
               module_set: str = "all") -> Dict[str, IndexLoRALinear]:
    """Index-resident wrappers holding the index slots of all ``ads`` (``serving/_common.py:294-306``):
    per layer, (n_adapters, L, n_blocks) int32 stacks of A and B and the pools in ``dtype``."""
    pa, pb = (p.to(device=device, dtype=dtype) for p in cb.twin_pools(ads[0].block_size, ads[0].n_bits,
                                                                     ads[0].sigma_a, ads[0].sigma_b))
    scale = float(ads[0].alpha) / ads[0].rank
    paths = [m["name"] for m in ads[0].modules]

    def factory(path, lin):
        ia = torch.stack([torch.from_numpy(np.asarray(ad.indices[path]["A"]).astype(np.int32)) for ad in ads])
        ib = torch.stack([torch.from_numpy(np.asarray(ad.indices[path]["B"]).astype(np.int32)) for ad in ads])
        return IndexLoRALinear(lin, ia.to(device), ib.to(device), pa, pb, ads[0].rank, scale)

    return wrap_linears(model, select_paths(paths, module_set), factory)


def set_assign(wrapped: Dict[str, nn.Module], assign: Optional[torch.Tensor]) -> None:
    """Route sample i of every wrapped linear to slot ``assign[i]`` (``serving/_common.py:309-311``)."""
    for mod in wrapped.values():
        mod.assign = assign


class SharedInputGroup:
    """Bank-backed layers whose linears read the same input (the q / k / v projections).

    The first member called with an input computes every member's base output, adds all
    their deltas in one grouped call whose members share one shrink over x
    (``lithe_lora_delta_grouped``: one shrink and one expand launch), returns its own and
    keeps the others until their members are called with the same input tensor (the same
    object at the same version counter, under the same routing tensor and bank generation; an
    inference-mode tensor has no version counter, so an in-place write into it between its members'
    calls is not seen).
    Any other call recomputes the group and drops what was pending, so results never depend on
    the call order.
    """

    def __init__(self, layers: Sequence[IndexLoRALinear]):
        if len(layers) < 2 or any(l._bank is None for l in layers):
            raise ValueError("a shared-input group needs two or more bank-backed layers")
        bank = layers[0]._bank[0]
        if any(l._bank[0] is not bank or l.rank != layers[0].rank or l.base.in_features != layers[0].base.in_features
               for l in layers):
            raise ValueError("grouped layers must share one bank, rank and input width")
        self.layers = list(layers)
        self._key = None
        self._pending: List[Optional[torch.Tensor]] = [None] * len(layers)

    def _compute(self, x: torch.Tensor) -> List[torch.Tensor]:
        lead = self.layers[0]
        outs = [l.base(x) for l in self.layers]
        squeeze = x.dim() == 2
        x3 = (x.unsqueeze(1) if squeeze else x).contiguous()
        o3 = [(o.unsqueeze(1) if squeeze else o) for o in outs]
        o3 = [o if o.is_contiguous() else o.contiguous() for o in o3]
        slots = (torch.zeros((x3.shape[0], 1), dtype=torch.int32, device=x.device) if lead.assign is None
                 else lead.assign.to(device=x.device, dtype=torch.int32).reshape(-1, 1).contiguous())
        # one grouped call: the members share one shrink job over x (one launch for the shrink,
        # one for every member's expand)
        _grouped_delta([x3] * len(self.layers), o3, lead._bank[0].words, [l._bank[1] for l in self.layers],
                       [l._bank[2] for l in self.layers], lead.pool_a, lead.pool_b, slots, lead.rank,
                       [l.scaling for l in self.layers])
        return [o.squeeze(1) if squeeze else o for o in o3]

    def _state(self, x: torch.Tensor):
        """What the pending outputs were computed from, besides the input object itself: its
        version, the routing tensor and its version, and the bank's generation (bumped by every
        write into a slot)."""
        a = self.layers[0].assign
        return (_hip.version_of(x), id(a), _hip.version_of(a) if isinstance(a, torch.Tensor) else None,
                self.layers[0]._bank[0].generation)

    def output(self, i: int, x: torch.Tensor) -> torch.Tensor:
        state = self._state(x)
        same = self._key is not None and self._key[0]() is x and self._key[1] == state
        if same and self._pending[i] is not None:
            out, self._pending[i] = self._pending[i], None
            return out
        outs = self._compute(x)
        self._key = (weakref.ref(x), state)
        self._pending = [o if j != i else None for j, o in enumerate(outs)]
        return outs[i]


class SharedInputMember(nn.Module):
    """Stands in for one layer of a ``SharedInputGroup`` (same ``base``, ``assign`` and slots)."""

    def __init__(self, group: SharedInputGroup, index: int):
        super().__init__()
        self.layer = group.layers[index]
        self._group = group
        self._index = index

    @property
    def base(self) -> nn.Linear:
        return self.layer.base

    @property
    def assign(self):
        return self.layer.assign

    @assign.setter
    def assign(self, value):
        self.layer.assign = value

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._group.output(self._index, x)


# The independent linears of each stage of a FLUX block, in call order: a serving step can compute
# a stage's base outputs and then add all of its deltas in one grouped call.
STAGES = {
    "proj": ("attn.to_q", "attn.to_k", "attn.to_v", "attn.add_q_proj", "attn.add_k_proj", "attn.add_v_proj"),
    "out": ("attn.to_out.0", "attn.to_add_out"),
    "up": ("ff.net.0.proj", "ff_context.net.0.proj"),
    "down": ("ff.net.2", "ff_context.net.2"),
}


class StageGroup:
    """Bank-backed layers of one block stage whose deltas run as one grouped call.

    ``group(inputs)`` returns ``[layer_m.base(inputs[m]) + delta_m]`` for every member m: the base
    GEMMs first, then one ``lithe_lora_delta_grouped`` launch pair over the whole stage (members
    given the same input tensor, e.g. q / k / v, share its shrink). Routing is the first member's
    ``assign`` (``set_assign`` gives every member the same).
    """

    def __init__(self, layers: Sequence[IndexLoRALinear]):
        layers = [getattr(l, "layer", l) for l in layers]      # shared-input stand-ins carry their layer
        if not 1 <= len(layers) <= _hip.MAX_GROUP_MODULES or any(l._bank is None for l in layers):
            raise ValueError(f"a stage group holds 1 to {_hip.MAX_GROUP_MODULES} bank-backed layers")
        bank = layers[0]._bank[0]
        if any(l._bank[0] is not bank or l.rank != layers[0].rank for l in layers):
            raise ValueError("grouped layers must share one bank and rank")
        self.layers = layers

    def __call__(self, inputs: Sequence[torch.Tensor]) -> List[torch.Tensor]:
        if len(inputs) != len(self.layers):
            raise ValueError(f"{len(self.layers)} inputs expected, got {len(inputs)}")
        lead = self.layers[0]
        bank = lead._bank[0]
        squeeze = inputs[0].dim() == 2
        outs = [l.base(x) for l, x in zip(self.layers, inputs)]
        xs, ys = [], []
        for i, (x, o) in enumerate(zip(inputs, outs)):
            if (x.dim() == 2) != squeeze or x.shape[0] != inputs[0].shape[0]:
                raise ValueError("every input must have the batch size and rank of the first")
            # one contiguous 3-D view per distinct input tensor, so shared shrinks stay shared
            first = next(j for j in range(i + 1) if inputs[j] is x)
            xs.append(xs[first] if first < i else (x.unsqueeze(1) if squeeze else x).contiguous())
            ys.append(o.unsqueeze(1) if squeeze else o)
        bsz = xs[0].shape[0]
        slots = (torch.zeros((bsz, 1), dtype=torch.int32, device=xs[0].device) if lead.assign is None
                 else lead.assign.to(device=xs[0].device, dtype=torch.int32).reshape(-1, 1).contiguous())
        _grouped_delta(xs, ys, bank.words, [l._bank[1] for l in self.layers], [l._bank[2] for l in self.layers],
                       lead.pool_a, lead.pool_b, slots, lead.rank, [l.scaling for l in self.layers])
        return outs


def stage_groups(wrapped: Dict[str, nn.Module]) -> Dict[Tuple[str, str], StageGroup]:
    """The FLUX block stages among bank-backed wrappers: {(block prefix, stage): StageGroup} for
    every stage of ``STAGES`` whose linears are all wrapped (a single block's q / k / v form its
    "proj" stage), members in call order."""
    groups: Dict[Tuple[str, str], StageGroup] = {}
    for path in wrapped:
        for stage, suffixes in STAGES.items():
            if not path.endswith(suffixes[0]):
                continue
            prefix = path[: -len(suffixes[0])]
            full = [prefix + s for s in suffixes]
            if all(m in wrapped for m in full):
                groups[(prefix, stage)] = StageGroup([wrapped[m] for m in full])
            elif stage == "proj" and all(m in wrapped for m in full[:3]) and not any(m in wrapped for m in full[3:]):
                groups[(prefix, stage)] = StageGroup([wrapped[m] for m in full[:3]])
    return groups


class AttentionGroup:
    """The six projections of a FLUX double-block attention (image ``to_q`` / ``to_k`` / ``to_v``
    over ``hidden_states``, text ``add_q_proj`` / ``add_k_proj`` / ``add_v_proj`` over
    ``encoder_hidden_states``) added in one grouped call when the attention module is entered.

    A forward pre-hook on the attention module reads the two inputs it is called with (keyword or
    positional, as diffusers' ``Attention`` takes them), computes the six base outputs and their
    deltas with one ``StageGroup`` call (the image and text projections each share a shrink), and
    keeps each output for its projection. A projection called with the input its output was
    computed from (same tensor object and version, same routing tensor and version, same bank
    generation) takes it; any other call runs the projection's own per-module forward, so results
    never depend on how the attention uses its projections. Eager mode: the pending state lives in
    Python (``torch.compile`` users keep the per-layer ops).
    """

    def __init__(self, attn: nn.Module, layers: Sequence[IndexLoRALinear]):
        if len(layers) != 6:
            raise ValueError("an attention group holds the six q / k / v projections of both streams")
        self.stage = StageGroup(layers)
        self.layers = self.stage.layers
        self._pending: List[Optional[tuple]] = [None] * 6
        self.calls = 0      # grouped calls made (one per attention entry with both inputs)
        self.handle = attn.register_forward_pre_hook(self._enter, with_kwargs=True)

    def _state(self, x: torch.Tensor):
        a = self.layers[0].assign
        return (_hip.version_of(x), id(a), _hip.version_of(a) if isinstance(a, torch.Tensor) else None,
                self.layers[0]._bank[0].generation)

    def _enter(self, module, args, kwargs):
        h = kwargs.get("hidden_states", args[0] if len(args) > 0 else None)
        c = kwargs.get("encoder_hidden_states", args[1] if len(args) > 1 else None)
        self._pending = [None] * 6
        if not isinstance(h, torch.Tensor) or not isinstance(c, torch.Tensor) or h.shape[0] != c.shape[0]:
            return None
        inputs = [h, h, h, c, c, c]
        outs = self.stage(inputs)
        self.calls += 1
        self._pending = [(weakref.ref(x), self._state(x), o) for x, o in zip(inputs, outs)]
        return None

    def output(self, i: int, x: torch.Tensor) -> torch.Tensor:
        p = self._pending[i]
        if p is not None and p[0]() is x and p[1] == self._state(x):
            self._pending[i] = None
            return p[2]
        return self.layers[i](x)


class AttentionMember(nn.Module):
    """Stands in for one projection of an ``AttentionGroup`` (same ``base``, ``assign`` and slots)."""

    def __init__(self, group: AttentionGroup, index: int):
        super().__init__()
        self.layer = group.layers[index]
        self._group = group
        self._index = index

    @property
    def base(self) -> nn.Linear:
        return self.layer.base

    @property
    def assign(self):
        return self.layer.assign

    @assign.setter
    def assign(self, value):
        self.layer.assign = value

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._group.output(self._index, x)


def wrap_bank(model: nn.Module, bank: PackedBank, module_set: str = "all", dtype: Optional[torch.dtype] = None,
              fuse_shared_inputs: bool = False, group_attention: bool = False) -> Dict[str, nn.Module]:
    """Bank-backed index-resident wrappers for every linear named in the bank's layout.

    ``group_attention``: the six projections of every attention module that has both streams
    wrapped run as one grouped call when the module is entered (``AttentionGroup``).
    ``fuse_shared_inputs``: the q / k / v of every other shared input (single blocks, or double
    blocks without ``group_attention``) run as one ``SharedInputGroup``."""
    paths = select_paths(bank.layout.names, module_set)
    wrapped = wrap_linears(model, paths, lambda p, lin: IndexLoRALinear.from_bank(lin, bank, p, dtype))
    if group_attention:
        for path in list(wrapped):
            names = STAGES["proj"]
            if not path.endswith(names[0]):
                continue
            prefix = path[: -len(names[0])]
            members = [prefix + n for n in names]
            if not all(m in wrapped and isinstance(wrapped[m], IndexLoRALinear) for m in members):
                continue
            attn = model.get_submodule((prefix + names[0]).rsplit(".", 1)[0])
            group = AttentionGroup(attn, [wrapped[m] for m in members])
            for i, m in enumerate(members):
                wrapped[m] = AttentionMember(group, i)
                replace_module(model, m, wrapped[m])
    if fuse_shared_inputs:
        for path in list(wrapped):
            for names in SHARED_INPUT_GROUPS:
                if not path.endswith(names[0]):
                    continue
                prefix = path[: -len(names[0])]
                members = [prefix + n for n in names]
                if not all(m in wrapped and isinstance(wrapped[m], IndexLoRALinear) for m in members):
                    continue
                group = SharedInputGroup([wrapped[m] for m in members])
                for i, m in enumerate(members):
                    wrapped[m] = SharedInputMember(group, i)
                    replace_module(model, m, wrapped[m])
    return wrapped


def wrap_decoded(model: nn.Module, paths: Sequence[str], kernel: str = "sgmv") -> Dict[str, PerSampleLoRALinear]:
    """Decoded-mode wrappers (``serving/_common.py:268-269``)."""
    return wrap_linears(model, paths, lambda p, lin: PerSampleLoRALinear(lin, kernel))


def install_per_sample(wrapped: Dict[str, PerSampleLoRALinear], decoded: Sequence[Dict]) -> None:
    """Point every wrapped linear at the factors of ``decoded[i]`` for slot i (``serving/_common.py:272-275``)."""
    for path, mod in wrapped.items():
        mod.set_factors([d[path] for d in decoded], per_sample=True)


def install_single(wrapped: Dict[str, PerSampleLoRALinear], decoded: Dict) -> None:
    """One adapter for every sample (``serving/_common.py:278-280``)."""
    for path, mod in wrapped.items():
        mod.set_factors([decoded[path]], per_sample=False)


def install_decoded_bank(wrapped: Dict[str, PerSampleLoRALinear], bank: PackedBank, slots) -> Dict:
    """Decode-on-swap: the selected bank slots decoded in one launch, installed as every
    layer's stacked factors (factor pair i = ``slots[i]``; set ``assign`` to pick pairs)."""
    st = bank.decode_stacked(slots)
    n = len(list(slots))
    for path, mod in wrapped.items():
        a, b = st[path]
        mod.set_stacked(a, b, torch.full((n,), bank.layout.scaling, dtype=torch.float32, device=a.device))
    return st
